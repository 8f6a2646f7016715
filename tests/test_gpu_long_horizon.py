"""BASELINE configs 3 and 4 at their stated lengths against the CPU oracle in
glibc mode (gpu).

The fixtures tests/golden/long_horizon_<arm>.npz hold the oracle's
trajectory (ORC_LIBM: the reference's arithmetic with glibc's expf/log1pf)
for the 24-layer synthetic GDN-1.3B from a zero state: a 4096-token uniform
prompt, then teacher-forced steps over the fixed 4096-token stream (4096
steps for the BF16 arms, 1024 for the FP32 control arm);
tests/golden/make_long_horizon.py wrote them.  The engine runs the same
trajectory and is held to the north star's gates:

  arm            argmax agreement    logits max |err|    final state rel-L2
  bf16w_fp32s    >= 99.9 % of steps  <= 2e-2             <= 1e-3
  ref            >= 99.9 % of steps  <= 2e-2             <= 1e-3
  fp32           100 % of steps      <= 1e-4             <= 1e-3

The logit error is taken over the oracle's 16 largest logits of every
teacher step and over all 32000 logits at three steps (the fixture keeps
those); the state error over every 128th value of the final recurrent state.
The engine evaluates glibc's transcendental methods exactly (gdn_libm.h), so
the trajectory is expected to equal the fixture bit for bit, which is
asserted as well.  At 8 steps spread over the teacher phase the oracle also
restarts from the engine's state and must reproduce that step's logits,
argmax and next state bit for bit.
"""
import os

import numpy as np
import pytest

import gateddeltanet_amd as g

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
GOLDEN = os.path.join(HERE, "golden")
ARMS = {
    # arm: (engine contract, oracle contract, BF16 weights, argmax floor, logit bound)
    "bf16w_fp32s": (g.CONTRACT_BF16W_FP32S, 1, True, 0.999, 2e-2),
    "ref": (g.CONTRACT_REF, 0, True, 0.999, 2e-2),
    "fp32": (g.CONTRACT_FP32, 2, False, 1.0, 1e-4),
}
STATE_BOUND = 1e-3
RESTARTS = 8


def same_bits(a, b):
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    nan = np.isnan(a) & np.isnan(b)
    return a.shape == b.shape and bool(((a.view(np.uint32) == b.view(np.uint32)) | nan).all())


@pytest.mark.parametrize("arm", list(ARMS))
def test_long_horizon_gates(orc, arm):
    path = os.path.join(GOLDEN, f"long_horizon_{arm}.npz")
    fx = np.load(path)  # numeric arrays only (allow_pickle stays False)
    contract, orc_contract, bf16, floor, bound = ARMS[arm]
    _, _, prompt_len, steps, stride, _, topk = (int(v) for v in fx["meta"])
    print(f"[long-horizon {arm}] prompt {prompt_len} + {steps} teacher steps", flush=True)
    model = g.Model.synth(num_layers=24, seed=0, std=0.02, bf16=bf16)
    rs = g.RunState(model, contract)
    try:
        prompt = g.synth_tokens(prompt_len, 0, 1, 32000)
        stream = g.synth_tokens(4096, 0, 2, 32000)
        pa, _, _ = rs.teacher_forced(prompt, prompt_len, timing=False)
        prompt_agree = float((pa == fx["prompt_argmax"]).mean())
        rec, _ = rs.save_state()
        pp = fx["post_prompt_state"]
        pp_rel = float(np.linalg.norm(rec[::stride] - pp) / np.linalg.norm(pp))
        print(f"[long-horizon {arm}] prompt argmax agreement {prompt_agree:.5f}, "
              f"post-prompt state rel-L2 {pp_rel:.3e}", flush=True)

        restart_at = set(np.linspace(0, steps - 1, RESTARTS).astype(int).tolist())
        hdr = orc.header_from(model.config)
        argmax = np.zeros(steps, np.int32)
        exact_steps = 0
        worst_top = 0.0
        worst_full = 0.0
        full = {int(s): i for i, s in enumerate(fx["full_steps"])}
        restarts_ok = 0
        for s in range(steps):
            tok = int(stream[s % stream.size])
            if s in restart_at:
                before_rec, before_conv = rs.save_state()
            argmax[s] = rs.decode_step(tok)
            logits = rs.logits()
            top = logits[fx["topk_idx"][s]]
            worst_top = max(worst_top, float(np.abs(top - fx["topk_val"][s]).max()))
            exact_steps += int(same_bits(top, fx["topk_val"][s]))
            if s in full:
                worst_full = max(worst_full, float(np.abs(logits - fx["full_logits"][full[s]]).max()))
            if s in restart_at:
                st, cv = before_rec.copy(), before_conv.copy()
                want, want_logits, _ = orc.decode_step(orc_contract, hdr, model.blob, st, cv, tok, orc.LIBM)
                after_rec, after_conv = rs.save_state()
                assert want == argmax[s], (arm, s)
                assert same_bits(logits, want_logits), (arm, s)
                assert same_bits(after_rec, st) and same_bits(after_conv, cv), (arm, s)
                restarts_ok += 1
            if (s + 1) % 1024 == 0:
                print(f"[long-horizon {arm}] step {s + 1}/{steps}", flush=True)
        rec, _ = rs.save_state()
    finally:
        rs.free()
        model.free()
    agree = float((argmax == fx["argmax"]).mean())
    fs = fx["final_state"]
    rel = float(np.linalg.norm(rec[::stride] - fs) / np.linalg.norm(fs))
    print(f"[long-horizon {arm}] teacher argmax agreement {agree:.5f} "
          f"({int((argmax != fx['argmax']).sum())} of {steps} differ), logits max|err| top-{topk} "
          f"{worst_top:.3e}, full {worst_full:.3e}, final state rel-L2 {rel:.3e}, "
          f"steps with bit-exact top-{topk} logits {exact_steps}/{steps}, "
          f"oracle restarts bit-exact {restarts_ok}/{RESTARTS}", flush=True)
    assert restarts_ok == RESTARTS
    assert agree >= floor, agree
    assert max(worst_top, worst_full) <= bound, (worst_top, worst_full)
    assert rel <= STATE_BOUND, rel
    # glibc's transcendentals reproduced exactly: the whole trajectory is the
    # reference's
    assert agree == 1.0 and exact_steps == steps and worst_full == 0.0 and rel == 0.0
    assert (pa == fx["prompt_argmax"]).all()
