#!/usr/bin/env python3
"""Benchmark of the quantized projection hot path on one MI355X.

Workload: the Qwen2.5-0.5B projection set at M=1 over 24 layers -- q
896->896, k/v 896->128, o 896->896, gate/up 896->4864, down 4864->896 -- symmetric int4 with an
f32 scale per 32 weights, x ~ N(0, 1), random N(0, 0.02) weights (synthetic; no checkpoint).
One step streams every projection once. Inputs are resident in HBM before timing starts.

Reported:
  value            GB/s of the batched launch (two launches per step: the 144 K=896 matrices,
                   then the 24 K=4864 ones), cold: 3 weight replicas rotate (672 MB > the
                   256 MB Infinity Cache), algorithmic bytes / wall time of the timed steps;
  sequential_*     the same step as 168 per-projection launches in one hipGraph (the
                   reference's dispatch order), cold;
  lm_head          config 2: the 151936 x 896 int8 tied head with the fused greedy argmax (and
                   its finalize launch), the head GEMV launch alone, and the sampled token;
  per_gemv_us      single launches of each shape, cold;
  roofline         the dominant kernel (the K=896 batched launch), its algorithmic bytes over
                   its own HIP-event-timed duration on the library's stream;
  prefill          config 3: the bf16-MFMA prefill GEMM at M = 256 / 128 (gate and down
                   shapes) in TFLOP/s and % of the 2.5 PFLOP/s bf16 peak, and the chunk's
                   f16-MFMA flash attention at the start and the end of a 2048 context;
  decode           config 4: greedy tok/s at 2048 context (graph and eager, with and without
                   the per-token readback);
  cpu_baseline     the reference's CPU loop (linearQ4, quant.ts:95-111) as restated by the
                   oracle, on a bounded sample, host cores stated.

Usage: python bench.py [--gpus 1] [--steps 30] [--warmup 5]
"""

from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "int4 GEMV achieved HBM GB/s (% of 8 TB/s); decode tok/s at 2048 ctx"
HBM_PEAK_GBS = 8000.0
HIDDEN, INTER, KV, LAYERS, VOCAB = 896, 4864, 128, 24, 151936
GROUP = 32
# (name, rows, K) per layer, in decode order (graph_decode.ts:276-353)
PROJECTIONS = [("q", HIDDEN, HIDDEN), ("k", KV, HIDDEN), ("v", KV, HIDDEN), ("o", HIDDEN, HIDDEN),
               ("gate", INTER, HIDDEN), ("up", INTER, HIDDEN), ("down", HIDDEN, INTER)]


def gemv_bytes(rows: int, k: int, bits: int = 4, group: int = GROUP) -> int:
    """Algorithmic bytes of one decode GEMV: codes + f32 scales + x read + y written."""
    return rows * k * bits // 8 + rows * (k // group) * 4 + k * 4 + rows * 4


STEP_BYTES = LAYERS * sum(gemv_bytes(r, k) for _, r, k in PROJECTIONS)
BATCH896_BYTES = LAYERS * sum(gemv_bytes(r, k) for n, r, k in PROJECTIONS if k == HIDDEN)
LM_HEAD_BYTES = VOCAB * HIDDEN + VOCAB * 4 + HIDDEN * 4 + VOCAB * 4


class HipEvents:
    """hipEvent timing on a given stream (the library's own)."""

    def __init__(self):
        self.hip = ctypes.CDLL("libamdhip64.so")
        self.hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]

    def create(self):
        e = ctypes.c_void_p()
        assert self.hip.hipEventCreate(ctypes.byref(e)) == 0
        return e

    def record(self, e, stream):
        assert self.hip.hipEventRecord(e, ctypes.c_void_p(stream)) == 0

    def sync(self, e):
        assert self.hip.hipEventSynchronize(e) == 0

    def ms(self, a, b) -> float:
        out = ctypes.c_float()
        assert self.hip.hipEventElapsedTime(ctypes.byref(out), a, b) == 0
        return out.value


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def make_projection_set():
    from enargeia_amd import quant

    mats = []
    for layer in range(LAYERS):
        for slot, (name, rows, k) in enumerate(PROJECTIONS):
            w = quant.normal(rows * k, 0x5EED ^ (layer * 16 + slot), 0.02)
            mats.append((name, quant.quantize_sym(w, rows, k, 4, GROUP)))
    return mats


def make_replica(dev, mats, out) -> dict:
    """One copy of the projection set on the device and the step's two batched plans: every
    K=896 matrix (q, k, v, o, gate, up of the 24 layers: 144 segments) in one plan and every
    K=4864 one (down: 24 segments) in the other, each matrix writing its rows at its offset in
    `out` (the order of `mats`)."""
    from enargeia_amd import kernels as K

    bufs, seg896, seg4864, singles = [], [], [], []
    off = 0
    for name, q in mats:
        bp, bs = dev.upload(q.packed), dev.upload(q.scales)
        bufs += [bp, bs]
        seg = (bp, bs, None, None, out, q.rows, off)
        (seg896 if q.cols == HIDDEN else seg4864).append(seg)
        singles.append((name, q, bp, bs, off))
        off += q.rows
    plans = (K.GemvPlan(dev, HIDDEN, GROUP, seg896), K.GemvPlan(dev, INTER, GROUP, seg4864))
    return {"bufs": bufs, "plans": plans, "singles": singles}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--replicas", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--decode-profile", action="store_true",
                    help="only the config-4 decode steps, launched eagerly (for rocprofv3 kernel statistics of a "
                         "decode step; graph capture is left out of profiled runs)")
    ap.add_argument("--prefill-profile", action="store_true",
                    help="only the config-3 prefill GEMM and chunk-attention launches (for rocprofv3 kernel "
                         "statistics of those kernels)")
    ap.add_argument("--prompt-profile", action="store_true",
                    help="only the prompt path (eg_decoder_prefill of a 2048-token prompt as one chunk and in chunks "
                         "of 256) on the config-4 model, for rocprofv3 kernel statistics of the prompt chain")
    ap.add_argument("--head-profile", action="store_true",
                    help="only the config-2 LM head (fused argmax) and sampled-token calls, for rocprofv3 kernel "
                         "statistics of the head and the sampler")
    ap.add_argument("--skip-decode", action="store_true",
                    help="leave out the config-4 decode measurement (rocprofv3 kernel tracing does not survive the "
                         "decoder's captured graph; --decode-profile covers the decode step eagerly)")
    ap.add_argument("--decode-timeline", action="store_true",
                    help="only the config-4 decode step captured in a hipGraph, with per-wave wall-clock stamps "
                         "(eg_test_launch_stamps): the per-launch timeline of the step as it is timed")
    ap.add_argument("--traffic-probe", action="store_true",
                    help="only launch the dominant kernel and two calibration kernels of known size "
                         "(for rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE runs)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported (the path is "
              "single-GPU; see DESIGN.md for how it would shard)", file=sys.stderr)
        return 2

    from enargeia_amd import kernels as K
    from enargeia_amd import quant

    if args.traffic_probe:
        return traffic_probe()
    if args.prefill_profile:
        dev = K.Device(0)
        print(json.dumps(prefill_numbers(dev, HipEvents(), dev.stream, args)), flush=True)
        dev.close()
        return 0
    if args.prompt_profile:
        from enargeia_amd.model import QWEN25_05B, Decoder, DeviceModel, synthetic_model
        dev = K.Device(0)
        dm = DeviceModel(dev, synthetic_model(QWEN25_05B))
        dec = Decoder(dm)
        print(json.dumps(prompt_throughput(dev, dec, QWEN25_05B)), flush=True)
        dec.close()
        dm.release()
        dev.close()
        return 0
    if args.head_profile:
        dev = K.Device(0)
        print(json.dumps(head_numbers(dev, HipEvents(), dev.stream, args, np.random.default_rng(7))), flush=True)
        dev.close()
        return 0
    if args.decode_timeline:
        from enargeia_amd import _lib
        _lib.use_profiling_build()  # the stamps live in the profiling build only
        dev = K.Device(0)
        print(json.dumps(decode_timeline(dev, args)), flush=True)
        dev.close()
        return 0
    if args.decode_profile:
        dev = K.Device(0)
        ev = HipEvents()
        print(json.dumps(decode_throughput(dev, ev, dev.stream, args, modes=("eager",))), flush=True)
        dev.close()
        return 0
    t0 = time.time()
    mats = make_projection_set()
    log(f"quantized {len(mats)} projection matrices in {time.time() - t0:.1f}s")

    dev = K.Device(0)
    ev = HipEvents()
    stream = dev.stream
    R = args.replicas

    rng = np.random.default_rng(7)
    x896 = dev.upload(rng.standard_normal(HIDDEN, dtype=np.float32))
    x4864 = dev.upload(rng.standard_normal(INTER, dtype=np.float32))
    rows_total = sum(q.rows for _, q in mats)
    out = dev.buffer(rows_total * 4)

    # ---- weights: R replicas, each with its own plans and per-op graph ----
    replicas = [make_replica(dev, mats, out) for _ in range(R)]
    log(f"uploaded {R} replicas of {STEP_BYTES / 1e6:.1f} MB")

    dec = K.ComputeKernel(dev, K.with_format(K.MATMUL_Q4_DECODE, 4, K.ENC_SIGNED))
    zero_bias = dev.buffer(INTER * 4)

    def per_op(rep):
        for name, q, bp, bs, off in rep["singles"]:
            u = dec.uniform()
            u.write(K.matmul_q4_dims(1, q.rows, q.cols, False, GROUP, q.rows, off))
            xin = x896 if q.cols == HIDDEN else x4864
            dec.encode(dec.bind_group([xin, bp, bs, None, zero_bias, out, u]), (1, 1, 1))

    def batched(rep):
        rep["plans"][0].launch(x896)
        rep["plans"][1].launch(x4864)

    def timed(fn, n):
        """ms per call of fn(i) over n back-to-back calls, one event pair around all of them."""
        a, b = ev.create(), ev.create()
        ev.record(a, stream)
        for i in range(n):
            fn(i)
        ev.record(b, stream)
        ev.sync(b)
        return ev.ms(a, b) / n

    # ---- batched step (value): eager stream launches, and the same two launches captured in
    # one hipGraph per replica (how a decode loop replays its step) ----
    # The GPU idles through the host-side model build; back-to-back steps for ~0.5 s bring its
    # clocks up before anything is timed (the first timed bursts otherwise read 10-25% slow).
    t_ramp = time.perf_counter()
    while time.perf_counter() - t_ramp < 0.5:
        for i in range(50):
            batched(replicas[i % R])
        dev.sync()
    for i in range(args.warmup):
        batched(replicas[i % R])
    dev.sync()
    eager_ms = timed(lambda i: batched(replicas[i % R]), args.steps)
    step_graphs = []
    for rep in replicas:
        dev.capture_begin()
        batched(rep)
        step_graphs.append(dev.capture_end())
    for i in range(args.warmup):
        step_graphs[i % R].launch()
    graph_ms = timed(lambda i: step_graphs[i % R].launch(), args.steps)
    step_ms = min(eager_ms, graph_ms)
    step_launch = "hipGraph" if graph_ms <= eager_ms else "stream"
    value = STEP_BYTES / (step_ms * 1e-3) / 1e9
    log(f"batched step: {eager_ms * 1e3:.1f} us eager, {graph_ms * 1e3:.1f} us as a graph -> {value:.0f} GB/s cold")

    # the dominant kernel alone: back-to-back launches over the cold replicas, one event pair
    # around the burst, so the per-launch average is the kernel's own duration
    burst = 3 * args.steps
    for i in range(R):
        replicas[i]["plans"][0].launch(x896)
    dominant_ms = timed(lambda i: replicas[i % R]["plans"][0].launch(x896), burst)
    log(f"K=896 batched launch alone: {dominant_ms * 1e3:.1f} us ({BATCH896_BYTES / dominant_ms / 1e6:.0f} GB/s)")
    down_ms = timed(lambda i: replicas[i % R]["plans"][1].launch(x4864), burst)
    down_bytes = STEP_BYTES - BATCH896_BYTES
    log(f"K=4864 batched launch alone: {down_ms * 1e3:.1f} us ({down_bytes / down_ms / 1e6:.0f} GB/s)")

    # warm: the same replica every step (226 MB, under the 256 MB Infinity Cache); enough steps
    # first that the cache holds what it will hold
    for _ in range(30):
        batched(replicas[0])
    warm_ms = timed(lambda i: batched(replicas[0]), args.steps)
    warm_gbs = STEP_BYTES / (warm_ms * 1e-3) / 1e9
    log(f"batched warm: {warm_ms * 1e3:.1f} us/step, {warm_gbs:.0f} GB/s")

    # ---- per-op sequential step in a hipGraph ----
    graphs = []
    for rep in replicas:
        dev.capture_begin()
        per_op(rep)
        graphs.append(dev.capture_end())
    for i in range(args.warmup):
        graphs[i % R].launch()
    ss, se = ev.create(), ev.create()
    ev.record(ss, stream)
    for i in range(args.steps):
        graphs[i % R].launch()
    ev.record(se, stream)
    ev.sync(se)
    seq_ms = ev.ms(ss, se) / args.steps
    seq_gbs = STEP_BYTES / (seq_ms * 1e-3) / 1e9
    log(f"per-op graph: {seq_ms * 1e3:.1f} us/step, {seq_gbs:.0f} GB/s cold")

    # ---- single GEMV launches per shape (cold: rotate layers and replicas) ----
    per_gemv = {}
    for shape_name in ("q", "k", "gate", "down"):
        cands = [(rep, s) for rep in replicas for s in rep["singles"] if s[0] == shape_name]
        times = []
        for j, (rep, (name, q, bp, bs, off)) in enumerate(cands[: 3 * LAYERS]):
            u = dec.uniform()
            u.write(K.matmul_q4_dims(1, q.rows, q.cols, False, GROUP, q.rows, off))
            a, b = ev.create(), ev.create()
            xin = x896 if q.cols == HIDDEN else x4864
            ev.record(a, stream)
            dec.encode(dec.bind_group([xin, bp, bs, None, zero_bias, out, u]), (1, 1, 1))
            ev.record(b, stream)
            ev.sync(b)
            if j >= 2:
                times.append(ev.ms(a, b))
        us = float(np.median(times)) * 1e3
        nbytes = gemv_bytes(q.rows, q.cols)
        per_gemv[f"{shape_name}_{q.rows}x{q.cols}"] = {"us": round(us, 2), "gbs": round(nbytes / (us * 1e-6) / 1e9, 1)}
    log(f"per-GEMV: {per_gemv}")

    for g in graphs + step_graphs:
        g.destroy()
    for rep in replicas:
        for p in rep["plans"]:
            p.destroy()
        for b in rep["bufs"]:
            b.release()

    hn = head_numbers(dev, ev, stream, args, rng)
    head_us, head_gbs, sampled_us = hn["us"], hn["gbs"], hn["sampled_us"]
    head_gemv_gbs = LM_HEAD_BYTES / (hn["gemv_us"] * 1e-6) / 1e9

    # ---- prefill chunk (config 3) ----
    prefill = prefill_numbers(dev, ev, stream, args)

    # ---- decode tok/s at 2048 context (config 4) ----
    decode = None if args.skip_decode else decode_throughput(dev, ev, stream, args)

    # ---- roofline: the dominant kernel = the K=896 batched launch ----
    t896_ms = dominant_ms
    achieved = BATCH896_BYTES / (t896_ms * 1e-3) / 1e9
    traffic, traffic_commit = measured_traffic()
    roofline = {"bound": "hbm", "kernel": "gemv_kernel<4,SIGNED,...,BATCHED> (K=896 projections, 24 layers)",
                "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                "traffic_source": "not measured in this run: the committed rocprofv3 --pmc summary "
                                  "profiles/gemv_batched_config1_traffic.md (FETCH_SIZE + WRITE_SIZE per "
                                  "dispatch, each scaled by a calibration kernel of known size), measured on the "
                                  f"kernels of commit {traffic_commit}",
                "bytes_per_launch": BATCH896_BYTES, "avg_launch_us": round(t896_ms * 1e3, 2)}

    cpu = None if args.no_cpu_baseline else cpu_baseline(mats)
    dev.close()

    line = {
        "metric": METRIC, "value": round(value, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(step_ms, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32", "data": "synthetic (random N(0,0.02) weights, N(0,1) inputs)",
        "config": {"workload": "BASELINE config 1: Qwen2.5-0.5B projection set, 24 layers x 7 int4 GEMVs at M=1",
                   "format": "int4 symmetric, f32 scale per 32 along K", "bytes_per_step": STEP_BYTES,
                   "cache": f"cold: {R} rotating weight replicas ({R * STEP_BYTES / 1e6:.0f} MB)",
                   "launches_per_step": 2, "launch": step_launch},
        "step_us": {"eager": round(eager_ms * 1e3, 2), "graph": round(graph_ms * 1e3, 2),
                    "k896_launch": round(dominant_ms * 1e3, 2), "k4864_launch": round(down_ms * 1e3, 2)},
        "pct_of_peak": round(100 * value / HBM_PEAK_GBS, 2),
        "warm_gbs": round(warm_gbs, 1),
        "sequential_gbs": round(seq_gbs, 1), "sequential_us_per_step": round(seq_ms * 1e3, 1),
        "sequential_launches_per_step": LAYERS * len(PROJECTIONS),
        "lm_head": {"config": "BASELINE config 2: 151936x896 int8 per-row + fused argmax", "us": round(head_us, 2),
                    "gbs": round(head_gbs, 1), "pct_of_peak": round(100 * head_gbs / HBM_PEAK_GBS, 2),
                    "bytes": LM_HEAD_BYTES,
                    "gemv_alone": {"us": round(hn["gemv_us"], 2), "gbs": round(head_gemv_gbs, 1),
                                   "pct_of_peak": round(100 * head_gemv_gbs / HBM_PEAK_GBS, 2),
                                   "note": "the head GEMV launch alone (logits stored, no argmax): the decode-shape "
                                           "int8 GEMV; `us` above adds the argmax finalize launch"},
                    "sampled_token_us": round(sampled_us, 2),
                    "sampled_token_fused_us": round(hn["sampled_fused_us"], 2),
                    "dense_tables": dict(hn["dense"], config="the same head over an f16 / f32 table "
                                                             "(lm_head_f16 / lm_head_f32), GEMV alone"),
                    "sampled_config": "LM head + sampler, T 0.7 / top-p 0.9 / penalty 1.1, 512-id history: "
                                      "sampled_token_us through the reference's two ops (lm_head_q8, sample), "
                                      "sampled_token_fused_us through eg_lm_head_sample (the head hands the "
                                      "sampler its per-workgroup max and normaliser partials)"},
        "per_gemv_us": per_gemv,
        "prefill": prefill,
        "decode_tok_s_2048": decode["tok_s"] if decode else None,
        "decode": decode,
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


DECODE_STEPS = 128


GOLDEN_DECODE = os.path.join(ROOT, "tests", "golden", "config4_decode.npz")


def verify_decode_tokens(tokens: list, first_step: int) -> dict:
    """Compares the greedy tokens of the timed steps with the CPU oracle's run of the same
    workload (tests/golden/config4_decode.npz): tokens[i] is the output of workload step
    first_step + i. A step counts when the oracle's top-2 gap exceeds 1e-2 x rms(logits); a
    differing token at a near-tie ends the comparison (later steps then see other inputs)."""
    with np.load(GOLDEN_DECODE, allow_pickle=False) as g:
        want, gaps, rms = g["tokens"], g["gaps"], g["rms"]
    compared = mismatches = near_ties = 0
    diverged_at = None
    for i, tok in enumerate(tokens):
        s = first_step + i
        if gaps[s] > 1e-2 * rms[s]:
            compared += 1
            if tok != int(want[s]):
                mismatches += 1
                break
        else:
            near_ties += 1
            if tok != int(want[s]):
                diverged_at = s
                break
    return {"oracle": "tests/golden/config4_decode.npz", "compared": compared, "mismatches": mismatches,
            "near_ties": near_ties, "diverged_at_near_tie": diverged_at,
            "verified": mismatches == 0}


def head_numbers(dev, ev, stream, args, rng) -> dict:
    """the 151,936 x 896 int8 tied head with the fused greedy argmax (its
    finalize launch included), cold over 3 table replicas, and the sampled token (the head storing
    logits, then the sampler at T 0.7 / top-p 0.9 / penalty 1.1 over a 512-id history): the median
    time between events recorded after each of back-to-back calls."""
    from enargeia_amd import kernels as K
    from enargeia_amd import quant

    # ---- LM head (config 2), fused argmax, cold over 3 table replicas ----
    table = quant.quantize_sym(quant.normal(VOCAB * HIDDEN, 0x5EED ^ 0x1000, 0.02), VOCAB, HIDDEN, 8, HIDDEN)
    heads = [(dev.upload(table.packed), dev.upload(table.scales)) for _ in range(3)]
    del table
    h = dev.upload(rng.standard_normal(HIDDEN, dtype=np.float32))
    logits = dev.buffer(VOCAB * 4)
    res = dev.buffer(8)
    dims = K.embedding_dims(1, HIDDEN, 0, VOCAB, HIDDEN, VOCAB, 0)
    for i in range(args.warmup):
        K.lm_head_argmax(dev, h, heads[i % 3][0], heads[i % 3][1], None, logits, res, dims, 8, K.ENC_SIGNED)
    hs = [ev.create() for _ in range(args.steps + 1)]
    ev.record(hs[0], stream)
    for i in range(args.steps):
        K.lm_head_argmax(dev, h, heads[i % 3][0], heads[i % 3][1], None, logits, res, dims, 8, K.ENC_SIGNED)
        ev.record(hs[i + 1], stream)
    ev.sync(hs[-1])
    head_times = [ev.ms(hs[i], hs[i + 1]) for i in range(args.steps)]
    head_us = float(np.median(head_times)) * 1e3
    head_gbs = LM_HEAD_BYTES / (head_us * 1e-6) / 1e9
    log(f"lm_head+argmax: {head_us:.1f} us, {head_gbs:.0f} GB/s cold")

    # sampled token (config 2: T 0.7, top-p 0.9, penalty 1.1 over 512 ids): LM head + sampler
    smp = K.ComputeKernel(dev, K.SAMPLE)
    hist = dev.upload(rng.integers(0, VOCAB, 512).astype(np.uint32))
    tok = dev.buffer(16)
    head_k = K.ComputeKernel(dev, K.embedding_head_spec("q8", K.ENC_SIGNED))

    def sampled_token(i):
        hu = head_k.uniform()
        hu.write(dims)
        head_k.encode(head_k.bind_group([h, heads[i % 3][0], heads[i % 3][1], None, logits, hu]), (1, 1, 1))
        su = smp.uniform()
        su.write(K.sample_dims(VOCAB, 512, K.SamplingParams(0.7, 0.9, 1.1), (i * 0.618) % 1.0))
        smp.encode(smp.bind_group([logits, hist, tok, su]), (1, 1, 1))

    for i in range(args.warmup):
        sampled_token(i)
    ss2 = [ev.create() for _ in range(args.steps + 1)]
    ev.record(ss2[0], stream)
    for i in range(args.steps):
        sampled_token(i)
        ev.record(ss2[i + 1], stream)
    ev.sync(ss2[-1])
    sampled_us = float(np.median([ev.ms(ss2[i], ss2[i + 1]) for i in range(args.steps)])) * 1e3
    log(f"lm_head+sample (T 0.7, top-p 0.9, penalty 1.1): {sampled_us:.1f} us")

    # the same sampled token through eg_lm_head_sample: the head applies the penalty and hands the
    # sampler its per-workgroup (max, index, normaliser) partials (the decoder's sampled steps)
    def fused_token(i):
        K.lm_head_sample(dev, h, heads[i % 3][0], heads[i % 3][1], None, logits, hist, tok, dims,
                         K.sample_dims(VOCAB, 512, K.SamplingParams(0.7, 0.9, 1.1), (i * 0.618) % 1.0), 8,
                         K.ENC_SIGNED)

    for i in range(args.warmup):
        fused_token(i)
    ss4 = [ev.create() for _ in range(args.steps + 1)]
    ev.record(ss4[0], stream)
    for i in range(args.steps):
        fused_token(i)
        ev.record(ss4[i + 1], stream)
    ev.sync(ss4[-1])
    fused_us = float(np.median([ev.ms(ss4[i], ss4[i + 1]) for i in range(args.steps)])) * 1e3
    log(f"lm_head_sample, one call (same parameters): {fused_us:.1f} us")

    # the head GEMV alone (the reference's lm_head_q8 binding: logits stored, no argmax)
    def plain_head(i):
        hu = head_k.uniform()
        hu.write(dims)
        head_k.encode(head_k.bind_group([h, heads[i % 3][0], heads[i % 3][1], None, logits, hu]), (1, 1, 1))

    for i in range(args.warmup):
        plain_head(i)
    ss3 = [ev.create() for _ in range(args.steps + 1)]
    ev.record(ss3[0], stream)
    for i in range(args.steps):
        plain_head(i)
        ev.record(ss3[i + 1], stream)
    ev.sync(ss3[-1])
    plain_us = float(np.median([ev.ms(ss3[i], ss3[i + 1]) for i in range(args.steps)])) * 1e3
    log(f"lm_head GEMV alone: {plain_us:.1f} us, {LM_HEAD_BYTES / (plain_us * 1e-6) / 1e9:.0f} GB/s cold")
    for a, b in heads:
        a.release()
        b.release()

    # the same head shape over an f16 and an f32 table (the reference's 'f16' / 'f32' embedding
    # dtypes): the head GEMV alone, one table (272 / 545 MB, past the 256 MB Infinity Cache)
    dense = {}
    for dtype, bits in (("f16", 16), ("f32", 32)):
        t = quant.dense_table(quant.normal(VOCAB * HIDDEN, 0x5EED ^ 0x1000, 0.02), VOCAB, HIDDEN, bits)
        bt = dev.upload(t.packed)
        nbytes = t.packed.nbytes + HIDDEN * 4 + VOCAB * 4
        del t
        dk = K.ComputeKernel(dev, K.embedding_head_spec(dtype))

        def dense_head(i):
            hu = dk.uniform()
            hu.write(dims)
            dk.encode(dk.bind_group([h, bt, None, None, logits, hu]), (1, 1, 1))

        for i in range(args.warmup):
            dense_head(i)
        es = [ev.create() for _ in range(args.steps + 1)]
        ev.record(es[0], stream)
        for i in range(args.steps):
            dense_head(i)
            ev.record(es[i + 1], stream)
        ev.sync(es[-1])
        us = float(np.median([ev.ms(es[i], es[i + 1]) for i in range(args.steps)])) * 1e3
        dense[dtype] = {"us": round(us, 2), "gbs": round(nbytes / (us * 1e-6) / 1e9, 1), "bytes": nbytes}
        log(f"lm_head_{dtype} GEMV: {us:.1f} us, {dense[dtype]['gbs']:.0f} GB/s")
        bt.release()
    return {"us": head_us, "gbs": head_gbs, "sampled_us": sampled_us, "sampled_fused_us": fused_us, "gemv_us": plain_us,
            "dense": dense}


def decode_throughput(dev, ev, stream, args, modes=("eager", "graph")) -> dict:
    """the Qwen2.5-0.5B-shaped model (synthetic weights, int4 g32 projections,
    int8 tied head, f16 KV cache) on the workload of enargeia_amd.model.config4_workload: cache
    rows [0, 1888) random f16 (the reference's prime-then-decode method, decode.test.ts:97-118),
    a 32-token prompt at positions 1888..1919 (untimed), then 128 greedy steps at positions
    1920..2047, timed. One step = the whole token: embedding, 24 layers, LM head, argmax. tok_s
    includes the one 4-byte readback per token (Session.decodeStep's rule); device_tok_s chains
    the steps on the device with no readback. The timed steps' tokens are checked against the CPU
    oracle's run of the same workload."""
    from enargeia_amd.model import QWEN25_05B, Decoder, DeviceModel, cache_fill, config4_workload, synthetic_model

    cfg = QWEN25_05B
    w = config4_workload(cfg)
    assert w.steps == DECODE_STEPS and w.prime + len(w.prompt) + w.steps == cfg.max_context
    t0 = time.time()
    host = synthetic_model(cfg)
    dm = DeviceModel(dev, host)
    del host
    dec = Decoder(dm)
    kf, vf = cache_fill(cfg, w.fill_seed)
    dev.write(dec.buffers.k_cache, kf.view(np.uint16))
    dev.write(dec.buffers.v_cache, vf.view(np.uint16))
    dev.sync()
    del kf, vf
    log(f"decode model ready in {time.time() - t0:.1f}s")
    start = w.prime + len(w.prompt)
    result = {"config": "BASELINE config 4: Qwen2.5-0.5B shape, 24 layers, int4 g32 + int8 tied head, f16 KV",
              "context": cfg.max_context, "prompt": len(w.prompt), "steps": DECODE_STEPS,
              "positions": [start, cfg.max_context - 1], "launches_per_token": 5 * cfg.layers + 2}
    for mode in modes:
        if mode == "graph":
            dec.capture()
        # the prompt (untimed): each token at its position, the last one's argmax is the first input
        for i, t in enumerate(w.prompt):
            dec.reset(w.prime + i, t)
            first = dec.step(read_token=True)
        # warm-up: steps at positions start.. (rewritten identically by the timed steps)
        for _ in range(8):
            dec.step(read_token=False)
        dec.reset(start, first)
        a, b = ev.create(), ev.create()
        t = time.perf_counter()
        ev.record(a, stream)
        tokens = [dec.step(read_token=True) for _ in range(DECODE_STEPS)]
        ev.record(b, stream)
        ev.sync(b)
        wall = time.perf_counter() - t
        result[f"{mode}_tok_s"] = round(DECODE_STEPS / wall, 1)
        result[f"{mode}_ms_per_token"] = round(wall / DECODE_STEPS * 1e3, 4)
        result[f"{mode}_tokens_vs_oracle"] = verify_decode_tokens([first] + tokens, len(w.prompt) - 1)
        # device-chained: same steps, no per-token readback
        dec.reset(start, first)
        ev.record(a, stream)
        for _ in range(DECODE_STEPS):
            dec.step(read_token=False)
        ev.record(b, stream)
        ev.sync(b)
        result[f"{mode}_device_tok_s"] = round(DECODE_STEPS / (ev.ms(a, b) * 1e-3), 1)
        log(f"decode ({mode}): {result[f'{mode}_tok_s']} tok/s with a readback per token, "
            f"{result[f'{mode}_device_tok_s']} tok/s device-chained; tokens vs oracle "
            f"{result[f'{mode}_tokens_vs_oracle']}")
    best = max(modes, key=lambda m: result[f"{m}_tok_s"])
    result["tok_s"] = result[f"{best}_tok_s"]
    result["launch"] = best
    result["verified"] = all(result[f"{m}_tokens_vs_oracle"]["verified"] for m in modes)
    if "graph" in modes:
        # the reference's live default (ui/engine.ts:261): T 0.7 / top-p 0.9 / penalty 1.1 over the
        # session's history (the prompt and every token), one device-side draw per step; the same
        # positions, captured, one readback per token
        dec.set_sampling(0.7, 0.9, 1.1)  # recaptures the step with the sampler
        dec.seed(0x5EED)
        dec.set_history(list(w.prompt) + [first])
        dec.reset(start, first)
        for _ in range(8):
            dec.step(read_token=False)
        dec.set_history(list(w.prompt) + [first])
        dec.reset(start, first)
        t = time.perf_counter()
        sampled = [dec.step(read_token=True) for _ in range(DECODE_STEPS)]
        wall = time.perf_counter() - t
        result["sampled_tok_s"] = round(DECODE_STEPS / wall, 1)
        result["sampled_ms_per_token"] = round(wall / DECODE_STEPS * 1e3, 4)
        result["sampled_config"] = "T 0.7 / top-p 0.9 / penalty 1.1, history = prompt + tokens, graph"
        result["sampled_vs_oracle"] = verify_sampled(dec, w)
        log(f"decode (graph, sampled): {result['sampled_tok_s']} tok/s with a readback per token; "
            f"{len(set(sampled))} distinct tokens; vs oracle {result['sampled_vs_oracle']}")
        dec.set_sampling(0.0, 1.0, 1.0)
    if "graph" in modes:
        result["f32_cache"] = f32_cache_decode(dev, dm, cfg, w, first, [first] + tokens)
    result["prompt"] = prompt_throughput(dev, dec, cfg)
    step_bytes = (STEP_BYTES + LM_HEAD_BYTES
                  + 2 * cfg.layers * (start + DECODE_STEPS // 2) * cfg.kv_heads * cfg.head_dim * 2)
    result["gbs_at_best"] = round(step_bytes * result["tok_s"] / 1e9, 1)
    dec.close()
    dm.release()
    return result


def f32_cache_decode(dev, dm, cfg, w, first, f16_tokens) -> dict:
    """The same greedy steps on a decoder with the reference's f32 KV cache variant (SessionOptions
    cacheDType 'f32'): the primed rows [0, 1888) hold the f16 run's values as f32, the prompt and
    the 128 timed steps append unrounded rows; captured, one readback per token. The f32 cache's
    numerics are held to the oracle by tests/test_gpu_decode.py; here its tokens are counted
    against the f16 run's (they may part where the top two logits are closer than the f16
    rounding of the new rows moves them)."""
    from enargeia_amd.model import Decoder, cache_fill

    dec = Decoder(dm, cache="f32")
    try:
        kf, vf = cache_fill(cfg, w.fill_seed)
        dev.write(dec.buffers.k_cache, kf.astype(np.float32))
        dev.write(dec.buffers.v_cache, vf.astype(np.float32))
        dev.sync()
        del kf, vf
        dec.capture()
        for i, t in enumerate(w.prompt):
            dec.reset(w.prime + i, t)
            dec.step(read_token=True)
        start = w.prime + len(w.prompt)
        for _ in range(8):
            dec.step(read_token=False)
        dec.reset(start, first)
        t = time.perf_counter()
        tokens = [dec.step(read_token=True) for _ in range(DECODE_STEPS)]
        wall = time.perf_counter() - t
        same = sum(int(a == b) for a, b in zip([first] + tokens, f16_tokens))
        res = {"tok_s": round(DECODE_STEPS / wall, 1), "ms_per_token": round(wall / DECODE_STEPS * 1e3, 4),
               "tokens_equal_to_f16_run": f"{same}/{len(f16_tokens)}",
               "config": "config 4 greedy steps with an f32 KV cache (eg_decoder_create_cache), graph, "
                         "a readback per token"}
        log(f"decode (graph, f32 KV cache): {res['tok_s']} tok/s with a readback per token; "
            f"tokens equal to the f16 run {res['tokens_equal_to_f16_run']}")
        return res
    finally:
        dec.close()


GOLDEN_SAMPLED = os.path.join(ROOT, "tests", "golden", "config4_sampled.npz")


def verify_sampled(dec, w) -> dict:
    """The sampled-decoding check of tests/test_gpu_decode_config4_sampled.py on the timed decoder
    (captured step): the oracle's sampled run of config 4 (tests/golden/config4_sampled.npz: the
    prompt's last position, then 32 steps at T 0.1 / top-p 0.9 / penalty 1.1 from seed 0x5eed) -
    draws equal bit for bit at every step, the token equal to the oracle's sampler on the GPU's
    own logits wherever that sampler is 2e-6 clear of its boundaries, and to the oracle's token
    wherever its margins clear the logit error (4 x max error over its 64 largest logits / T)."""
    import oracle

    with np.load(GOLDEN_SAMPLED, allow_pickle=False) as f:
        g = {k: f[k] for k in f.files}
    T, top_p = float(g["temperature"]), float(g["top_p"])
    for s_, t in enumerate(w.prompt[:-1]):
        dec.reset(w.prime + s_, t)
        dec.step(read_token=False)
    dec.set_sampling(T, top_p, float(g["penalty"]))
    dec.seed(int(g["seed"]))
    history = [int(t) for t in w.prompt]
    dec.set_history(history)
    dec.reset(w.prime + len(w.prompt) - 1, w.prompt[-1])
    draws_equal, sampler, e2e, forced, max_err = 0, 0, 0, 0, 0.0
    steps = len(g["positions"])
    for i, pos in enumerate(g["positions"]):
        tok = dec.step()
        draws_equal += int(dec.sample_params()["random"].view(np.uint32) == g["draws"][i].view(np.uint32))
        got = dec.logits()
        err = float(np.abs(got[g["top_ids"][i]].astype(np.float64) - g["top_values"][i]).max())
        max_err = max(max_err, err / float(g["rms"][i]))
        mine, info, _ = oracle.sample(got, np.zeros(0, np.uint32), T, top_p, 1.0, float(g["draws"][i]))
        if info.bisect_margin > 2e-6 and info.draw_margin > 2e-6:
            sampler += int(tok == mine) - (tok != mine) * 1000  # a mismatch fails the check below
        want = int(g["tokens"][i])
        eps = 4 * err / T
        if g["bisect_margin"][i] > eps and g["draw_margin"][i] > eps:
            e2e += int(tok == want) - (tok != want) * 1000
        history.append(want)
        if tok != want:
            dec.reset(int(pos) + 1, want)
            dec.set_history(history)
            forced += 1
    return {"oracle": "tests/golden/config4_sampled.npz", "steps": steps, "draws_equal": draws_equal,
            "sampler_on_gpu_logits_equal": sampler, "end_to_end_equal": e2e, "continued_on_oracle_token": forced,
            "max_logit_error_vs_rms": round(max_err, 6),
            "verified": draws_equal == steps and sampler >= 0.8 * steps and e2e >= 0.75 * steps}


STAMP_WAVES = 8192  # per launch slot (eg_test_launch_stamps)


def decode_timeline(dev, args) -> dict:
    """The config-4 decode step as bench.py times it - captured in a hipGraph, at positions
    1920..2047, one 4-byte readback per token - with every launch writing per-wave wall-clock
    stamps (eg_test_launch_stamps: each wave's entry and exit, s_memrealtime). The stamps of the
    last of 8 back-to-back steps are read, so every sample follows seven steps run as the timed
    loop runs them. Per launch of the step: its duration (first wave in to last wave out) and the
    gap to the next launch, medians over the samples; the step's first-in to last-out time, and
    the host's share of a token (wall time of the 8 steps / 8 minus the step). Greedy steps, then
    the same positions sampled (T 0.7 / top-p 0.9 / penalty 1.1)."""
    from enargeia_amd import _lib
    from enargeia_amd.model import QWEN25_05B, Decoder, DeviceModel, cache_fill, config4_workload, synthetic_model

    lib = _lib.load()
    hip = ctypes.CDLL("libamdhip64.so")
    rate_khz = ctypes.c_int()
    assert hip.hipDeviceGetAttribute(ctypes.byref(rate_khz), 10017, 0) == 0  # hipDeviceAttributeWallClockRate
    tick_us = 1e3 / rate_khz.value
    cfg = QWEN25_05B
    w = config4_workload(cfg)
    dm = DeviceModel(dev, synthetic_model(cfg))
    dec = Decoder(dm)
    kf, vf = cache_fill(cfg, w.fill_seed)
    dev.write(dec.buffers.k_cache, kf.view(np.uint16))
    dev.write(dec.buffers.v_cache, vf.view(np.uint16))
    dev.sync()
    del kf, vf
    start = w.prime + len(w.prompt)
    layer_names = ["q|k|v GEMV (RMSNorm stage)", "attention", "o GEMV (combine stage)", "gate|up SwiGLU pair",
                   "down GEMV"]
    result = {"config": "BASELINE config 4 decode step at positions 1920..2047, captured, a readback per token",
              "wall_clock_mhz": rate_khz.value / 1e3}
    cap = 5 * cfg.layers + 3
    buf = dev.buffer(cap * STAMP_WAVES * 16)
    for mode in ("greedy", "sampled"):
        if mode == "sampled":
            dec.set_sampling(0.7, 0.9, 1.1)
            dec.seed(0x5EED)
        dev.zero(buf, cap * STAMP_WAVES * 16)
        _lib.check(lib.eg_test_launch_stamps(dev.ctx, ctypes.c_void_p(buf.ptr), cap, None), dev.ctx)
        dec.capture()
        rec = ctypes.c_uint32()
        _lib.check(lib.eg_test_launch_stamps(dev.ctx, None, 0, ctypes.byref(rec)), dev.ctx)
        n = rec.value
        tail_names = ["LM head (final-norm stage)"] + (["sampler"] if mode == "sampled" else []) + ["step tail"]
        persistent = n == 1 + len(tail_names)
        if persistent:  # the 24 layers as one launch (eg_layers.hip)
            names = ["decode layers (one persistent launch)"] + tail_names
        else:
            names = [f"L{l} {layer_names[j]}" for l in range(cfg.layers) for j in range(5)] + tail_names
        assert n == len(names), f"{n} launches took a slot, {len(names)} expected"
        for i, t in enumerate(w.prompt):
            dec.reset(w.prime + i, t)
            first = dec.step(read_token=True)
        if mode == "sampled":
            dec.set_history(list(w.prompt) + [first])
        durs, gaps, steps_us, walls, phase_adds = [], [], [], [], []
        for rep in range(max(4, min(args.steps, 120) // 8)):
            dec.reset(start + 8 * (rep % 12), first)
            t = time.perf_counter()
            for _ in range(8):
                dec.step(read_token=True)
            walls.append((time.perf_counter() - t) / 8 * 1e6)
            # the sample: one more step, after zeroing the persistent launch's per-phase maxima
            dev.zero(buf, STAMP_WAVES * 8, STAMP_WAVES * 8)
            dec.step(read_token=True)
            raw = np.frombuffer(dev.read(buf, n * STAMP_WAVES * 16), np.uint64).reshape(n, STAMP_WAVES, 2)
            waves = [r[:STAMP_WAVES // 2] if (persistent and i == 0) else r for i, r in enumerate(raw)]
            t0s = np.array([r[r[:, 0] > 0, 0].min() for r in waves], np.float64)
            t1s = np.array([r[r[:, 1] > 0, 1].max() for r in waves], np.float64)
            durs.append((t1s - t0s) * tick_us)
            gaps.append((t0s[1:] - t1s[:-1]) * tick_us)
            steps_us.append((t1s[-1] - t0s[0]) * tick_us)
            if persistent:
                # per phase: ~ the first workgroup past its wait, the last one past it, the last
                # arrival (the first layer's q|k|v waits for nothing: the launch's first wave)
                flat = raw[0].reshape(-1)[STAMP_WAVES:STAMP_WAVES + 4 * 5 * cfg.layers].reshape(-1, 4)
                first_in = np.where(flat[:, 0] > 0, (~flat[:, 0]).astype(np.float64), np.nan)
                last_in = flat[:, 1].astype(np.float64)
                ends = flat[:, 2].astype(np.float64)
                first_in[0] = last_in[0] = t0s[0]
                prev = np.concatenate([[t0s[0]], ends[:-1]])
                phase_adds.append(np.stack([ends - prev, first_in - prev, last_in - first_in, ends - last_in]) * tick_us)
        d = np.median(np.array(durs), axis=0)
        g = np.median(np.array(gaps), axis=0)
        per_kind = {}
        first_tail = 1 if persistent else 5 * cfg.layers
        if persistent:
            # [4, phases]: the phase's add to the launch (previous phase's last arrival to its
            # own), of which: to the first workgroup past the wait, from there to the last one
            # past it, from there to the last arrival; medians over samples, then layers (the
            # first layer's q|k|v, which waits for nothing, left out)
            adds = np.median(np.array(phase_adds), axis=0)
            keys = ["adds_us", "to_first_past_wait_us", "first_to_last_past_wait_us", "last_past_wait_to_last_arrival_us"]
            per_kind[names[0]] = {"us": round(float(d[0]), 2), "gap_after_us": round(float(g[0]), 2),
                                  "phases": {kind: {k: round(float(np.median(adds[i, j + (5 if j == 0 else 0)::5])), 2)
                                                    for i, k in enumerate(keys)}
                                             for j, kind in enumerate(layer_names)}}
        else:
            for j, kind in enumerate(layer_names):
                per_kind[kind] = {"us": round(float(np.median(d[j:5 * cfg.layers:5])), 2),
                                  "gap_after_us": round(float(np.median(g[j:5 * cfg.layers:5])), 2)}
        for i in range(first_tail, n):
            per_kind[names[i]] = {"us": round(float(d[i]), 2),
                                  "gap_after_us": round(float(g[i]), 2) if i < n - 1 else None}
        step_us, wall_us = float(np.median(steps_us)), float(np.median(walls))
        result[mode] = {
            "launches": n, "samples": len(durs), "per_launch": per_kind,
            "kernel_us_per_step": round(float(d.sum()), 1), "gaps_us_per_step": round(float(g.sum()), 1),
            "first_in_to_last_out_us": round(step_us, 1), "wall_us_per_token": round(wall_us, 1),
            "host_and_readback_us_per_token": round(wall_us - step_us, 1)}
        log(f"decode timeline ({mode}): {result[mode]}")
    dec.close()
    dm.release()
    buf.release()
    return result


def prompt_throughput(dev, dec, cfg) -> dict:
    """The prompt path (eg_decoder_prefill: chunks of 256 rows through the bf16-MFMA projections
    and the chunk attention, then the first token from the last row): the reference's prefill
    figures (README.md:41-44: 1105 tok/s at 128 tokens, 708 tok/s at 2048 chunked at 256, 219 ms
    to the first token of a 32-token prompt, on an M2). Wall time per call, host to first token
    id, median of 5 after a warm-up call; GREEDY."""
    out = {"config": "Qwen2.5-0.5B shape, 24 layers, prompt at position 0 as one chunk (and 2048 tokens in the "
                     "reference's chunks of 256), wall time to the first token id (one readback)",
           "reference_m2": {"prefill_128_tok_s": 1105, "prefill_2048_tok_s": 708, "ttft_32_ms": 219}}
    for n, chunk in ((32, 2048), (128, 2048), (2048, 2048), (2048, 256)):
        dec.set_prefill_chunk(chunk)
        prompt = [int(t) for t in np.random.default_rng(0x5EED + n).integers(0, cfg.vocab, n)]
        dec.prefill(0, prompt)
        times = []
        for _ in range(5):
            t = time.perf_counter()
            dec.prefill(0, prompt)
            times.append(time.perf_counter() - t)
        ms = float(np.median(times)) * 1e3
        key = f"prefill_{n}" if chunk >= n else f"prefill_{n}_chunk{chunk}"
        out[key] = {"ms": round(ms, 3), "tok_s": round(n / ms * 1e3, 1)}
    dec.set_prefill_chunk(2048)
    out["ttft_32_ms"] = out["prefill_32"]["ms"]
    log(f"prompt: {out}")
    return out


BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 / fp16 matrix peak


def prefill_numbers(dev, ev, stream, args) -> dict:
    """the prefill chunk as a dense contraction. X [M x 896] (M = 256, 128)
    through the int4 g32 gate (4864 x 896) and down (896 x 4864) weights on the bf16 MFMA GEMM
    (eg_matmul_q4_prefill), and the chunk's attention on the f16 MFMA flash kernel
    (eg_attention_prefill, 14 / 2 heads, head_dim 64) at the start of the context and at its
    end (keys up to 2048). Median per-launch time of `steps` launches; TFLOP/s counts the
    useful products only (2 M N K for the GEMM; 4 D per unmasked (query, key, head) for
    attention)."""
    import ctypes

    from enargeia_amd import _lib, kernels as K, quant

    rng = np.random.default_rng(17)
    res = {"config": "BASELINE config 3: X [M x 896] through int4 g32 gate 896->4864 and down 4864->896, "
                     "bf16 MFMA, f32 accumulate; chunk attention on f16 MFMA"}
    gate = quant.quantize_sym(quant.normal(INTER * HIDDEN, 0x5EED ^ 0x300, 0.02), INTER, HIDDEN, 4, GROUP)
    down = quant.quantize_sym(quant.normal(HIDDEN * INTER, 0x5EED ^ 0x301, 0.02), HIDDEN, INTER, 4, GROUP)
    kern = K.ComputeKernel(dev, K.with_format(K.MATMUL_Q4_PREFILL, 4, K.ENC_SIGNED))
    keep = []

    def timed_each(fn, n):
        marks = [ev.create() for _ in range(n + 1)]
        for _ in range(3):
            fn()
        ev.record(marks[0], stream)
        for i in range(n):
            fn()
            ev.record(marks[i + 1], stream)
        ev.sync(marks[-1])
        return float(np.median([ev.ms(marks[i], marks[i + 1]) for i in range(n)])) * 1e3

    for m in (256, 128):
        for name, q in (("gate", gate), ("down", down)):
            x = dev.upload(rng.standard_normal((m, q.cols), dtype=np.float32))
            bp, bs = dev.upload(q.packed), dev.upload(q.scales)
            out = dev.buffer(m * q.rows * 4)
            keep += [x, bp, bs, out]
            u = kern.uniform()
            u.write(K.matmul_q4_dims(m, q.rows, q.cols, False, GROUP, q.rows, 0))
            bg = kern.bind_group([x, bp, bs, None, None, out, u])
            us = timed_each(lambda: kern.encode(bg, (1, 1, 1)), args.steps)
            tf = 2.0 * m * q.rows * q.cols / (us * 1e-6) / 1e12
            res[f"gemm_{name}_m{m}"] = {"us": round(us, 2), "tflops": round(tf, 2),
                                        "pct_of_bf16_peak": round(100 * tf / BF16_PEAK_TFLOPS, 2)}
    log(f"prefill GEMM: {res}")

    class Dims(ctypes.Structure):
        _fields_ = [(n, ctypes.c_uint32) for n in ("queries", "keys", "query_begin", "heads", "kv_heads",
                                                   "head_dim", "max_context")] + [("theta", ctypes.c_float)]

    H, KVH, D, CTX, M = 14, 2, 64, 2048, 256
    q = dev.upload(rng.standard_normal((M, H * D), dtype=np.float32))
    kvb = [dev.upload(rng.standard_normal((M, KVH * D), dtype=np.float32)) for _ in range(2)]
    caches = [dev.upload(rng.standard_normal(CTX * KVH * D, dtype=np.float32).astype(np.float16).view(np.uint16))
              for _ in range(2)]
    qr, out = dev.buffer(M * H * D * 4), dev.buffer(M * H * D * 4)
    keep += [q, qr, out] + kvb + caches
    vp = ctypes.c_void_p
    for begin in (0, CTX - M):
        d = Dims(M, begin + M, begin, H, KVH, D, CTX, 1.0e6)

        def call():
            _lib.check(_lib.load().eg_attention_prefill(dev.ctx, vp(q.ptr), vp(kvb[0].ptr), vp(kvb[1].ptr),
                                                        vp(caches[0].ptr), vp(caches[1].ptr), vp(qr.ptr),
                                                        vp(out.ptr), ctypes.byref(d)), dev.ctx)

        us = timed_each(call, args.steps)
        pairs = H * sum(begin + i + 1 for i in range(M))
        tf = 4.0 * D * pairs / (us * 1e-6) / 1e12
        res[f"attention_m{M}_begin{begin}"] = {"us": round(us, 2), "tflops": round(tf, 3)}
    # the same chunk over an f32 cache (eg_attention_prefill_f32: exact rows, f32 FMAs)
    caches32 = [dev.upload(rng.standard_normal(CTX * KVH * D, dtype=np.float32)) for _ in range(2)]
    keep += caches32
    for begin in (0, CTX - M):
        d = Dims(M, begin + M, begin, H, KVH, D, CTX, 1.0e6)

        def call32():
            _lib.check(_lib.load().eg_attention_prefill_f32(dev.ctx, vp(q.ptr), vp(kvb[0].ptr), vp(kvb[1].ptr),
                                                            vp(caches32[0].ptr), vp(caches32[1].ptr), vp(qr.ptr),
                                                            vp(out.ptr), ctypes.byref(d)), dev.ctx)

        us = timed_each(call32, args.steps)
        pairs = H * sum(begin + i + 1 for i in range(M))
        tf = 4.0 * D * pairs / (us * 1e-6) / 1e12
        res[f"attention_f32_cache_m{M}_begin{begin}"] = {"us": round(us, 2), "tflops": round(tf, 3)}
    log(f"prefill attention: { {k: v for k, v in res.items() if k.startswith('attention')} }")
    for b in keep:
        b.release()
    return res


CALIBRATION_BYTES = 256 << 20
TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "gemv_batched_config1_traffic.md")


def measured_traffic():
    """(HBM bytes per launch of the dominant kernel, the commit whose kernels were measured), from
    the committed rocprofv3 --pmc summary (FETCH_SIZE + WRITE_SIZE per dispatch, each scaled by its
    calibration kernel); (None, None) without it."""
    traffic, commit = None, None
    try:
        with open(TRAFFIC_PROFILE) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    traffic = int(line.split(":", 1)[1].strip().replace(",", ""))
                elif line.startswith("traffic_measured_at:"):
                    commit = line.split(":", 1)[1].strip()
    except OSError:
        pass
    return traffic, commit


def traffic_probe() -> int:
    """Dispatches, in order: argmax over CALIBRATION_BYTES of floats (reads exactly that),
    a zero fill of CALIBRATION_BYTES (writes exactly that), then the K=896 batched projection
    launch three times over three cold replicas, then the K=4864 one likewise. Per-dispatch
    FETCH_SIZE / WRITE_SIZE of the calibration kernels give the counters' scale; see profiles/."""
    from enargeia_amd import kernels as K
    from enargeia_amd import quant

    dev = K.Device(0)
    big = dev.buffer(CALIBRATION_BYTES)
    dev.zero(big, CALIBRATION_BYTES)
    dev.sync()
    out8 = dev.buffer(16)
    am = K.ComputeKernel(dev, K.ARGMAX)
    u = am.uniform()
    u.write(K.argmax_dims(CALIBRATION_BYTES // 4, 0))
    am.encode(am.bind_group([big, out8, u]), (1, 1, 1))
    dev.sync()
    dev.zero(big, CALIBRATION_BYTES)
    dev.sync()
    rng = np.random.default_rng(7)
    for k in (HIDDEN, INTER):
        rows = [r for _, r, kk in PROJECTIONS if kk == k]
        mats = [quant.quantize_sym(quant.normal(r * k, 300 + 10 * (k == INTER) + i, 0.02), r, k, 4, GROUP)
                for i, r in enumerate(rows)]
        out = dev.buffer(LAYERS * sum(rows) * 4)
        x = dev.upload(rng.standard_normal(k, dtype=np.float32))
        plans = []
        for _ in range(3):
            segs, off = [], 0
            for _layer in range(LAYERS):
                for q in mats:
                    segs.append((dev.upload(q.packed), dev.upload(q.scales), None, None, out, q.rows, off))
                    off += q.rows
            plans.append(K.GemvPlan(dev, k, GROUP, segs))
        for p in plans:
            p.launch(x)
        dev.sync()
    print(json.dumps({"traffic_probe": True, "calibration_bytes": CALIBRATION_BYTES,
                      "batch896_bytes": BATCH896_BYTES, "batch4864_bytes": STEP_BYTES - BATCH896_BYTES}),
          flush=True)
    dev.close()
    return 0


def cpu_baseline(mats):
    """The reference's CPU GEMV loop (the oracle's restatement of linearQ4, quant.ts:95-111:
    per-element dequant, float64 accumulate) over the same config-1 step: once on one thread,
    then 4 times on every host core. GB/s of the same algorithmic bytes."""
    import oracle

    rng = np.random.default_rng(3)
    xs = {HIDDEN: rng.standard_normal(HIDDEN, dtype=np.float32), INTER: rng.standard_normal(INTER, dtype=np.float32)}
    oq = [oracle.QuantizedMatrix(q.rows, q.cols, q.block_size, 4, oracle.ENC_SIGNED, q.packed, q.scales, None)
          for _, q in mats]
    cores = len(os.sched_getaffinity(0))
    cores = min(cores, int(os.environ.get("OMP_NUM_THREADS", cores)))

    def run(threads, reps):
        t = time.perf_counter()
        for _ in range(reps):
            for q in oq:
                oracle.gemv_threads(xs[q.cols], q, None, threads)
        return (time.perf_counter() - t) / reps

    one = run(1, 1)
    many = run(cores, 4)
    log(f"cpu baseline: one step in {one * 1e3:.0f} ms on 1 core, {many * 1e3:.0f} ms on {cores} cores")
    return {"value": round(STEP_BYTES / many / 1e9, 3), "unit": "GB/s", "cores": cores, "kind": "port",
            "sample": f"the full config-1 step ({STEP_BYTES} B, 168 GEMVs): 1 run on 1 thread, 4 runs on "
                      f"{cores} threads; oracle restatement of the reference's linearQ4 loop",
            "single_core_gbs": round(STEP_BYTES / one / 1e9, 4),
            "step_ms_single_core": round(one * 1e3, 1), "step_ms_all_cores": round(many * 1e3, 1),
            "javascript": js_baseline()}


def js_baseline():
    """The reference's CPU loop in its own language: oracle/linear_q4_time.js (linearQ4 and
    dequantElement, quant.ts:77-111, restated in plain JavaScript) under the host's Node, one core,
    over one layer of config 1 (7 GEMVs, 9.41 MB) 20 times; None where no Node is installed."""
    import shutil
    import subprocess

    node = shutil.which("node") or shutil.which("nodejs")
    if not node:
        return None
    res = subprocess.run([node, os.path.join(ROOT, "oracle", "linear_q4_time.js"), "20"], capture_output=True,
                         text=True, timeout=120)
    if res.returncode != 0:
        log(f"js baseline failed: {res.stderr.strip()[-300:]}")
        return None
    r = json.loads(res.stdout.strip().splitlines()[-1])
    log(f"cpu baseline (JavaScript, Node {r['node']}, 1 core): {r['gbs']:.4f} GB/s")
    return {"value": round(r["gbs"], 4), "unit": "GB/s", "cores": 1, "node": r["node"],
            "sample": "one config-1 layer (q, k, v, o, gate, up, down: 9,410,048 B), 20 runs, "
                      "oracle/linear_q4_time.js",
            "step_ms": round(r["seconds"] * LAYERS * 1e3, 1)}


if __name__ == "__main__":
    sys.exit(main())
