"""Writes tests/golden/long_horizon_<arm>.npz: the CPU oracle's trajectory
for BASELINE configs 3 and 4 at their stated lengths.

Each arm runs the 24-layer GDN-1.3B synthetic model (seed 0, N(0, 0.02)
weights, norm weights 1; BF16-rounded for the BF16 arms, plain FP32 for the
control arm) from a zero recurrent/conv state:
  1. a 4096-token uniform prompt (gdn_synth_tokens seed 0, stream 1), one
     decode step per token, as bench.py builds its post-prompt state;
  2. teacher-forced steps over the fixed uniform 4096-token stream (seed 0,
     stream 2), consumed cyclically: 4096 steps for the BF16 arms, 1024 for
     the FP32 arm.
The oracle runs with glibc expf/log1pf (ORC_LIBM), i.e. the transcendentals
the reference's gdn_model.cpp calls.

Stored per arm (data only):
  prompt_argmax[4096], argmax[S]            the greedy token of every step
  topk_idx[S][16], topk_val[S][16]          the 16 largest logits of every
                                            teacher step (descending value,
                                            lower index first on ties)
  full_steps[3], full_logits[3][32000]      every logit at three teacher steps
  post_prompt_state, final_state            recurrent state [L][H][K][V]
                                            flattened, every 128th value
  final_state_norms[L*H]                    Frobenius norm of each head's
                                            final state (float64)
  final_conv                                conv tails, every 16th value

Run (about an hour on 8 cores):
  python tests/golden/make_long_horizon.py [arm ...]   # arms: bf16w_fp32s ref fp32
"""
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

import gateddeltanet_amd as g  # noqa: E402  (host synth only: no GPU call)
from oracle import oracle as O  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))
L, V, PROMPT, TOPK = 24, 32000, 4096, 16
STATE_STRIDE, CONV_STRIDE = 128, 16
ARMS = {
    # arm: (oracle contract, BF16 weights, teacher steps)
    "bf16w_fp32s": (O.BF16W_FP32S, True, 4096),
    "ref": (O.REF, True, 4096),
    "fp32": (O.FP32, False, 1024),
}


def topk(logits: np.ndarray, k: int):
    # descending value, lower index first among equal values
    order = np.lexsort((np.arange(logits.size), -logits.astype(np.float64)))[:k]
    return order.astype(np.int32), logits[order].astype(np.float32)


def run_arm(arm: str) -> None:
    contract, bf16, steps = ARMS[arm]
    model = g.Model.synth(num_layers=L, seed=0, std=0.02, bf16=bf16)
    hdr = O.header_from(model.config)
    blob = model.blob
    prompt = g.synth_tokens(PROMPT, 0, 1, V)
    stream = g.synth_tokens(4096, 0, 2, V)
    state = np.zeros(L * 8 * 256 * 256, np.float32)
    conv = np.zeros(L * 3 * 3 * 2048, np.float32)
    full_steps = np.array([0, steps // 2, steps - 1], np.int32)
    out = {
        "prompt_argmax": np.zeros(PROMPT, np.int32),
        "argmax": np.zeros(steps, np.int32),
        "topk_idx": np.zeros((steps, TOPK), np.int32),
        "topk_val": np.zeros((steps, TOPK), np.float32),
        "full_steps": full_steps,
        "full_logits": np.zeros((full_steps.size, V), np.float32),
    }
    t0 = time.time()
    for i, tok in enumerate(prompt):
        out["prompt_argmax"][i], _, _ = O.decode_step(contract, hdr, blob, state, conv, int(tok), O.LIBM)
        if (i + 1) % 512 == 0:
            print(f"[{arm}] prompt {i + 1}/{PROMPT} {time.time() - t0:.0f}s", flush=True)
    out["post_prompt_state"] = state[::STATE_STRIDE].copy()
    for s in range(steps):
        tok = int(stream[s % stream.size])
        out["argmax"][s], logits, _ = O.decode_step(contract, hdr, blob, state, conv, tok, O.LIBM)
        out["topk_idx"][s], out["topk_val"][s] = topk(logits, TOPK)
        hit = np.nonzero(full_steps == s)[0]
        if hit.size:
            out["full_logits"][hit[0]] = logits
        if (s + 1) % 512 == 0:
            print(f"[{arm}] teacher {s + 1}/{steps} {time.time() - t0:.0f}s", flush=True)
    out["final_state"] = state[::STATE_STRIDE].copy()
    out["final_state_norms"] = np.sqrt(
        (state.astype(np.float64).reshape(L * 8, -1) ** 2).sum(axis=1))
    out["final_conv"] = conv[::CONV_STRIDE].copy()
    out["meta"] = np.array([contract, int(bf16), PROMPT, steps, STATE_STRIDE, CONV_STRIDE, TOPK], np.int64)
    path = os.path.join(HERE, f"long_horizon_{arm}.npz")
    np.savez_compressed(path, **out)
    print(f"[{arm}] wrote {path} ({os.path.getsize(path)} bytes) in {time.time() - t0:.0f}s", flush=True)
    model.free()


def main() -> None:
    arms = sys.argv[1:] or list(ARMS)
    for arm in arms:
        run_arm(arm)


if __name__ == "__main__":
    main()
