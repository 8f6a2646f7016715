"""bench.py's command line without a GPU: more than one GPU is refused with
a message (this build measures one GPU), and the options that select the
other BASELINE legs are there."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def run_bench(*args):
    return subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *args], capture_output=True,
                          text=True, timeout=120, cwd=ROOT)


def test_more_than_one_gpu_is_refused_with_a_message():
    for n in ("2", "8"):
        r = run_bench("--gpus", n)
        assert r.returncode == 2
        assert "single-GPU" in r.stderr and "--gpus 1" in r.stderr
        assert r.stdout.strip() == ""  # no bench line


def test_options_for_every_leg():
    r = run_bench("--help")
    assert r.returncode == 0
    for opt in ("--steps", "--warmup", "--gpus", "--contract", "--config", "--streams", "--prefill",
                "--prefill-mode", "--eager", "--no-secondary", "--copy-calibration"):
        assert opt in r.stdout, opt
