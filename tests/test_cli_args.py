"""gdn_eval_amd's command line on the CPU: the refusals that happen while the
arguments are parsed, before any device call (the decode runs themselves are
in test_gpu_cli.py)."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CLI = os.path.join(ROOT, "gateddeltanet_amd", "gdn_eval_amd")


def run(*args):
    if not os.path.exists(CLI):
        pytest.skip("gdn_eval_amd is not built")
    return subprocess.run([CLI, *args], capture_output=True, text=True, timeout=60)


def test_help_lists_the_decode_flags():
    r = run("--help")
    assert r.returncode == 0
    for flag in ("--dump-state", "--save-gdnstate", "--interstep-delay-ms", "--logits-reference"):
        assert flag in r.stdout


@pytest.mark.parametrize("args, msg", [
    (("--ftz",), "--ftz is not supported"),
    (("--benchmark-tokens", "t.txt", "--dump-state", "s"), "apply to the decode run"),
    (("--interstep-delay-ms", "x"), "bad value for --interstep-delay-ms"),
    (("--interstep-delay-ms",), "--interstep-delay-ms requires a value"),
])
def test_refusals(args, msg):
    r = run("--synth=1", "--decode-from-state", "none.gdnstate", *args)
    assert r.returncode == 2 and msg in r.stderr


def test_prefill_refuses_decode_only_flags():
    r = run("--synth=1", "--prefill", "p.txt", "--dump-state", "o.gdnstate", "--save-gdnstate", "x")
    assert r.returncode == 2 and "apply to the decode run, not --prefill" in r.stderr
