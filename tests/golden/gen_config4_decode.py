"""Writes tests/golden/config4_decode.npz: BASELINE config 4 run through the CPU oracle.

The Qwen2.5-0.5B-shaped synthetic model (enargeia_amd.model.synthetic_model: int4 g32
projections, int8 per-row tied table), the f16 cache primed with random rows up to the
workload's prime position, a 32-token prompt, then 128 greedy steps to position 2047 -- the
reference's prime-then-decode parity run (test/parity/decode.test.ts:97-118) composed by
oracle.decode.OracleDecoder (graph_decode.ts:246-385 over test/reference/ops.ts). Records per
step the greedy token, the top-2 logit gap and the logits' rms, and at a few steps the logits at
every 61st id plus the 8 largest, so a GPU run is compared step by step without storing 608 KB
of logits per step. Takes a few minutes on 8 cores:

    python tests/golden/gen_config4_decode.py
"""

from __future__ import annotations

import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from enargeia_amd.model import QWEN25_05B, cache_fill, config4_workload, synthetic_model  # noqa: E402
from oracle.decode import OracleDecoder  # noqa: E402

OUT = os.path.join(HERE, "config4_decode.npz")
SAMPLE_STRIDE = 61
TOP = 8


def main() -> None:
    cfg = QWEN25_05B
    w = config4_workload(cfg)
    t0 = time.time()
    model = synthetic_model(cfg)
    ora = OracleDecoder(model)
    kf, vf = cache_fill(cfg, w.fill_seed)
    ora.k[:] = kf.astype(np.float32)
    ora.v[:] = vf.astype(np.float32)
    fill_check = np.array([kf.reshape(-1)[:4096].astype(np.float64).sum(), vf.reshape(-1)[-4096:].astype(np.float64).sum()])
    del kf, vf
    print(f"model and cache ready in {time.time() - t0:.0f}s", flush=True)

    positions, inputs, tokens, gaps, rmss = [], [], [], [], []
    sampled_steps, sampled_values, top_ids, top_values = [], [], [], []
    n_prompt = len(w.prompt)
    total = n_prompt + w.steps
    keep = {0, n_prompt - 1, n_prompt, n_prompt + w.steps // 2, total - 1}
    tok = None
    for s in range(total):
        pos = w.prime + s
        inp = w.prompt[s] if s < n_prompt else tok
        logits = ora.step(inp, pos)
        order = np.argsort(logits, kind="stable")
        best = int(np.argmax(logits))  # first index of the maximum: ties to the lower id
        second = float(np.max(np.delete(logits, best)))
        positions.append(pos)
        inputs.append(inp)
        tokens.append(best)
        gaps.append(float(logits[best]) - second)
        rmss.append(float(np.sqrt(np.mean(logits.astype(np.float64) ** 2))))
        if s in keep:
            sampled_steps.append(s)
            sampled_values.append(logits[::SAMPLE_STRIDE].copy())
            top_ids.append(order[-TOP:][::-1].astype(np.uint32))
            top_values.append(logits[order[-TOP:][::-1]])
        tok = best
        if s % 16 == 0 or s == total - 1:
            print(f"step {s} pos {pos} token {best} gap {gaps[-1]:.4f} ({time.time() - t0:.0f}s)", flush=True)
    np.savez_compressed(
        OUT, prime=np.uint32(w.prime), prompt=np.array(w.prompt, np.uint32), steps=np.uint32(w.steps),
        fill_seed=np.uint32(w.fill_seed), fill_check=fill_check, positions=np.array(positions, np.uint32),
        inputs=np.array(inputs, np.uint32), tokens=np.array(tokens, np.uint32), gaps=np.array(gaps),
        rms=np.array(rmss), sample_stride=np.uint32(SAMPLE_STRIDE), sampled_steps=np.array(sampled_steps, np.uint32),
        sampled_values=np.stack(sampled_values).astype(np.float32), top_ids=np.stack(top_ids),
        top_values=np.stack(top_values).astype(np.float32))
    print(f"wrote {OUT} ({os.path.getsize(OUT)} bytes) in {time.time() - t0:.0f}s")


if __name__ == "__main__":
    main()
