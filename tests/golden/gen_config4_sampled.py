"""Writes tests/golden/config4_sampled.npz: sampled decoding on BASELINE config 4, through the CPU oracle.

The config-4 workload of gen_config4_decode.py (the Qwen2.5-0.5B-shaped synthetic model, the f16
cache primed with random rows to position 1888, the 32-token prompt fed greedily), then the
session's sampled decoding as Session.generate runs it (session.ts:416-495): the history is the
prompt, the last prompt position takes the first mulberry32 draw from seed 0x5eed
(sampleFromPrefill), and every later step one more (decodeStep), each token sampled by
oracle.sample (sample.wgsl:143-332) at T 0.1 / top-p 0.9 / repetition penalty 1.1 over the history
and then appended to it. Records per sampled step the draw, the token, the sampler's margins
(bisection mass to topP, draw target to the nearest cumulative boundary, both relative to the kept
mass) and the 64 largest penalized logits with their ids, so a GPU run compares its draws bit for
bit, its logits where they decide the draw, and its token wherever the margins clear the logit
error. Takes a minute or two on 8 cores:

    python tests/golden/gen_config4_sampled.py
"""

from __future__ import annotations

import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402
from enargeia_amd.model import QWEN25_05B, cache_fill, config4_workload, synthetic_model  # noqa: E402
from oracle.decode import OracleDecoder  # noqa: E402

OUT = os.path.join(HERE, "config4_sampled.npz")
TEMPERATURE, TOP_P, PENALTY, SEED = 0.1, 0.9, 1.1, 0x5EED
SAMPLED_STEPS = 33  # the prompt's last position, then 32 decode steps
TOP = 64


def main() -> None:
    cfg = QWEN25_05B
    w = config4_workload(cfg)
    t0 = time.time()
    model = synthetic_model(cfg)
    ora = OracleDecoder(model)
    kf, vf = cache_fill(cfg, w.fill_seed)
    ora.k[:] = kf.astype(np.float32)
    ora.v[:] = vf.astype(np.float32)
    del kf, vf
    print(f"model and cache ready in {time.time() - t0:.0f}s", flush=True)

    n_prompt = len(w.prompt)
    for s in range(n_prompt - 1):
        ora.step(w.prompt[s], w.prime + s)
    draws = oracle.Mulberry32Stream(SEED)
    history = list(w.prompt)
    tok = w.prompt[-1]
    rec = {k: [] for k in ("positions", "draws", "tokens", "bisect_margin", "draw_margin", "top_ids", "top_values",
                           "rms")}
    for i in range(SAMPLED_STEPS):
        pos = w.prime + n_prompt - 1 + i
        logits = ora.step(tok, pos)
        r = np.float32(draws())
        tok, info, pen = oracle.sample(logits, np.array(history, np.uint32), TEMPERATURE, TOP_P, PENALTY, r)
        order = np.argsort(pen, kind="stable")[::-1][:TOP]
        rec["positions"].append(pos)
        rec["draws"].append(r)
        rec["tokens"].append(tok)
        rec["bisect_margin"].append(info.bisect_margin)
        rec["draw_margin"].append(info.draw_margin)
        rec["top_ids"].append(order.astype(np.uint32))
        rec["top_values"].append(pen[order])
        rec["rms"].append(float(np.sqrt(np.mean(pen.astype(np.float64) ** 2))))
        history.append(tok)
        print(f"sampled step {i} pos {pos} draw {r:.6f} token {tok} margins {info.bisect_margin:.2e} "
              f"{info.draw_margin:.2e} ({time.time() - t0:.0f}s)", flush=True)
    np.savez_compressed(
        OUT, prime=np.uint32(w.prime), prompt=np.array(w.prompt, np.uint32), fill_seed=np.uint32(w.fill_seed),
        temperature=np.float32(TEMPERATURE), top_p=np.float32(TOP_P), penalty=np.float32(PENALTY),
        seed=np.uint32(SEED), positions=np.array(rec["positions"], np.uint32),
        draws=np.array(rec["draws"], np.float32), tokens=np.array(rec["tokens"], np.uint32),
        bisect_margin=np.array(rec["bisect_margin"]), draw_margin=np.array(rec["draw_margin"]),
        top_ids=np.stack(rec["top_ids"]), top_values=np.stack(rec["top_values"]).astype(np.float32),
        rms=np.array(rec["rms"]))
    print(f"wrote {OUT} ({os.path.getsize(OUT)} bytes) in {time.time() - t0:.0f}s")


if __name__ == "__main__":
    main()
