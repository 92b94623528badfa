"""The prompt chain with the matrix-core path's roundings (test infrastructure only).

The reference encodes a prompt chunk (graph.ts:380-500: embed, then per layer RMSNorm, q / k / v
with biases, RoPE at positions begin + i, the cache append, causal attention over the cache,
o + residual, RMSNorm, SiLU(gate) * up, down + residual; the head on the last row) in f32. The
device chain runs the same operators with narrower operands, and this module restates the
chain with exactly those roundings, so that a test can hold the device to a bar set by f32
summation order rather than by bf16's unit roundoff:

  * every projection multiplies bf16(x) by bf16(the f32 dequantized weight), products exact,
    sums in float64, then bias or residual (eo_linear_q_bf16's model);
  * an RMSNorm before a projection (q | k | v, gate | up) is either folded into the projection's
    launch - x staged as bf16(h * w), each output row scaled by 1 / sqrt(mean(h^2) + eps) after
    the sums, then the bias - or run on its own (rmsnorm_rows: bf16(h * inv * w)) when the
    launch fills the device: the device folds it when the launch's tiles (64 rows x 64 columns;
    q | k | v: 18 column tiles at Qwen2.5-0.5B's shape, gate | up: 152 of 32 columns) number
    fewer than its CUs (256 on MI355X), so the choice follows the chunk's row count;
  * attention takes q after RoPE scaled by 1/8 (1/sqrt(64)) and rounded to f16, keys and values
    from the f16 cache, and walks the keys in tiles of 64 with a running max: per tile
    p = exp(s - max so far) rounded to f16 for the weighted sum of values, the sum of the
    unrounded p rescaled with the max; long key ranges split over workgroups as the device
    splits them (splits of whole tiles, each with its own running max, merged at the end);
  * SiLU(gate) * up in f32, rounded to bf16 as the down projection's x;
  * the head is the decode head (final RMSNorm, the int8 LM head GEMV with float64 sums).

The prompt runs in chunks of `chunk` rows, as the device's chain does.

``rounding="none"`` drops the bf16 and f16 operand roundings (the cache stays f16, as the
decoder's is): the chain is then the reference's prompt in f32 and equals OracleDecoder stepping
the same prompt one position at a time, which is how the chain's structure is pinned
(tests/test_oracle_chain.py): order of operators, residuals, RoPE positions, the causal mask,
the tile walk and the split merge. The operand roundings are pinned one by one: the bf16
projection against eo_linear_q_bf16, f16_array against binary16, and a one-key attention (p = 1
exactly, so the output is the value row whatever the rounding).

Only tests/ use it; the product never does.
"""

from __future__ import annotations

import numpy as np

from . import QuantizedMatrix, bf16_round_array, dequantize, gemv_threads, rmsnorm, rope
from .decode import _threads, dequant_row, f16_array


def _identity(a: np.ndarray) -> np.ndarray:
    return np.asarray(a, np.float32)


class _Weights:
    """Dequantized matrices of one model as float64, rounded to bf16 or not, built on first use."""

    def __init__(self, rounding: str, keep: bool = True):
        self.round = bf16_round_array if rounding == "device" else _identity
        self.keep = keep  # False: nothing is held between uses (a 24-layer model's would be ~3 GB)
        self.cache: dict[int, np.ndarray] = {}

    def __call__(self, q) -> np.ndarray:
        key = id(q)
        if key in self.cache:
            return self.cache[key]
        m = QuantizedMatrix(q.rows, q.cols, q.block_size, q.bits, q.encoding, np.asarray(q.packed, np.uint32),
                            np.asarray(q.scales, np.float32), None if q.zeros is None else np.asarray(q.zeros, np.uint32))
        # the device's f32 (code - zero) * scale, then its operand rounding
        w = self.round(dequantize(m).astype(np.float32)).astype(np.float64)
        if self.keep:
            self.cache[key] = w
        return w


def _linear(x: np.ndarray, q, bias, weights: _Weights, xround) -> np.ndarray:
    """[n, cols] -> [n, rows] f32: xround(x) . W^T in float64, plus the bias."""
    y = xround(x).astype(np.float64) @ weights(q).T
    if bias is not None:
        y = y + np.asarray(bias, np.float64)[None, :]
    return y.astype(np.float32)


def _linear_norm(h: np.ndarray, norm_w: np.ndarray, eps: float, q, bias, weights: _Weights, xround) -> np.ndarray:
    """RMSNorm(h) . W^T + bias with the norm folded in: xround(h * w) . W^T, each row then times
    1 / sqrt(mean(h^2) + eps) (f32), then the bias (f32)."""
    hw = (np.asarray(h, np.float32) * np.asarray(norm_w, np.float32)[None, :]).astype(np.float32)
    acc = (xround(hw).astype(np.float64) @ weights(q).T).astype(np.float32)
    h64 = np.asarray(h, np.float64)
    r = (1.0 / np.sqrt(np.mean(h64 * h64, axis=1, keepdims=True) + eps)).astype(np.float32)
    y = (acc * r).astype(np.float32)
    if bias is not None:
        y = (y + np.asarray(bias, np.float32)[None, :]).astype(np.float32)
    return y


KEY_TILE = 64          # keys per tile of the prefill attention
QUERY_BLOCK = 64       # queries per workgroup of it
SPLIT_TILES = 8        # a workgroup walks at most this many key tiles (split cap)
PARTIALS_BYTES = (64 << 20) - 8192  # the device's workspace for split partials


def attention_splits(queries: int, keys: int, heads: int, cu_count: int = 256) -> int:
    """Key tiles per split (0: no split) as the device chooses them: where the (query block, head)
    grid leaves CUs idle, splits of at least 4 tiles up to about one workgroup per CU, and so
    that no workgroup walks more than 8 tiles; bounded by the partials workspace."""
    blocks = (queries + QUERY_BLOCK - 1) // QUERY_BLOCK
    grid = blocks * heads
    tiles = (keys + KEY_TILE - 1) // KEY_TILE
    splits = 1
    if tiles >= 8:
        if grid < cu_count:
            splits = min((cu_count + grid - 1) // grid, tiles // 4)
        splits = max(splits, (tiles + SPLIT_TILES - 1) // SPLIT_TILES)
    rows = queries * heads
    while splits > 1 and splits * rows * (64 + 2) * 4 > PARTIALS_BYTES:
        splits -= 1
    return 0 if splits <= 1 else (tiles + splits - 1) // splits


def _walk(q: np.ndarray, K: np.ndarray, V: np.ndarray, limits: np.ndarray, kb: int, ke: int, pround):
    """One workgroup's walk over keys [kb, ke) in tiles of KEY_TILE for queries q [n, D] (query i
    sees keys <= limits[i]): (o unnormalised [n, D], running max m [n], sum l [n])."""
    n, D = q.shape
    m = np.full(n, -np.inf)
    l = np.zeros(n)
    o = np.zeros((n, D))
    for t0 in range(kb, ke, KEY_TILE):
        t1 = min(t0 + KEY_TILE, ke)
        s = q @ K[t0:t1].T
        s = np.where(np.arange(t0, t1)[None, :] <= limits[:, None], s, -np.inf)
        mnew = np.maximum(m, s.max(axis=1))
        live = np.isfinite(mnew)
        alpha = np.where(live & np.isfinite(m), np.exp(m - np.where(live, mnew, 0.0)), 0.0)
        p = np.where(live[:, None], np.exp(s - np.where(live, mnew, 0.0)[:, None]), 0.0)
        l = l * alpha + p.sum(axis=1)
        o = o * alpha[:, None] + pround(p.astype(np.float32)).astype(np.float64) @ V[t0:t1]
        m = np.where(live, mnew, m)
    return o, m, l


def _attention(qs: np.ndarray, k_cache: np.ndarray, v_cache: np.ndarray, begin: int, heads: int, kv_heads: int,
               head_dim: int, pround, cu_count: int = 256) -> np.ndarray:
    """Causal attention of the chunk's rows i (query at begin + i) over cache rows [0, begin + i].
    qs [n][heads*D] already scaled by 1/sqrt(D) (and rounded as the device rounds it); the caches
    [context][kv_heads][D]. Returns f32 [n][heads*D]."""
    n = qs.shape[0]
    group = heads // kv_heads
    end = begin + n
    q = qs.astype(np.float64).reshape(n, heads, head_dim)
    limits = begin + np.arange(n)
    skeys = attention_splits(n, end, heads, cu_count) * KEY_TILE
    out = np.empty((n, heads, head_dim), np.float64)
    for h in range(heads):
        K = k_cache[:end, h // group, :].astype(np.float64)
        V = v_cache[:end, h // group, :].astype(np.float64)
        if not skeys:
            o, _, l = _walk(q[:, h, :], K, V, limits, 0, end, pround)
            out[:, h, :] = o / l[:, None]
            continue
        parts = [_walk(q[:, h, :], K, V, limits, kb, min(kb + skeys, end), pround) for kb in range(0, end, skeys)]
        live = [np.isfinite(m) & (l > 0) for _, m, l in parts]
        M = np.max([np.where(lv, m, -np.inf) for (_, m, _), lv in zip(parts, live)], axis=0)
        acc = np.zeros((n, head_dim))
        L = np.zeros(n)
        for (o, m, l), lv in zip(parts, live):
            w = np.where(lv, np.exp(np.where(lv, m, 0.0) - M), 0.0)
            acc += o * w[:, None]
            L += l * w
        out[:, h, :] = acc / L[:, None]
    return out.reshape(n, heads * head_dim).astype(np.float32)


def _rmsnorm_rows(h: np.ndarray, norm_w: np.ndarray, eps: float) -> np.ndarray:
    """rmsnorm_rows' order: h * inv * w in f32, inv = 1 / sqrt(mean(h^2) + eps)."""
    h64 = np.asarray(h, np.float64)
    inv = (1.0 / np.sqrt(np.mean(h64 * h64, axis=1, keepdims=True) + eps)).astype(np.float32)
    return ((np.asarray(h, np.float32) * inv).astype(np.float32) * np.asarray(norm_w, np.float32)[None, :]).astype(np.float32)


def _projection(h, norm_w, eps, q, bias, w, xround, fold: bool) -> np.ndarray:
    if fold:
        return _linear_norm(h, norm_w, eps, q, bias, w, xround)
    return _linear(_rmsnorm_rows(h, norm_w, eps), q, bias, w, xround)


def _folds(rows: int, column_tiles: int, cu_count: int) -> bool:
    return column_tiles * ((rows + 63) // 64) < cu_count


def prefill_chain(model, prompt, begin: int, k_cache: np.ndarray, v_cache: np.ndarray, rounding: str = "device",
                  chunk: int = 256, cu_count: int = 256, weights: _Weights | None = None) -> np.ndarray:
    """The prompt `prompt` at positions begin.. through every layer, `chunk` rows at a time;
    returns the last row's logits (f32 [vocab]). k_cache / v_cache [layers][context][kv_heads][D]
    (f32 arrays holding f16 values) get the prompt's rows. rounding: "device" or "none"."""
    if rounding not in ("device", "none"):
        raise ValueError(f"rounding {rounding!r}")
    c = model.cfg
    H, D = c.hidden, c.head_dim
    w = weights or _Weights(rounding, keep=False)
    xround = bf16_round_array if rounding == "device" else _identity
    pround = f16_array if rounding == "device" else _identity
    qkv_tiles = (c.hidden + 2 * c.kv_heads * D + 63) // 64
    pair_tiles = (c.intermediate + 31) // 32
    h = None
    for c0 in range(0, len(prompt), chunk):
        ids = prompt[c0:c0 + chunk]
        n, pos = len(ids), begin + c0
        fold_qkv, fold_pair = _folds(n, qkv_tiles, cu_count), _folds(n, pair_tiles, cu_count)
        h = np.stack([dequant_row(model.embedding, int(t)) for t in ids]).astype(np.float32)
        for li, L in enumerate(model.layers):
            q = _projection(h, L.input_norm, c.rms_eps, L.mats["q"], L.biases["q"], w, xround, fold_qkv)
            k = _projection(h, L.input_norm, c.rms_eps, L.mats["k"], L.biases["k"], w, xround, fold_qkv)
            v = _projection(h, L.input_norm, c.rms_eps, L.mats["v"], L.biases["v"], w, xround, fold_qkv)
            qr = rope(q.reshape(-1), n, c.heads, D, c.rope_theta, pos).reshape(n, -1)
            kr = rope(k.reshape(-1), n, c.kv_heads, D, c.rope_theta, pos).reshape(n, -1)
            k_cache[li, pos:pos + n] = f16_array(kr).reshape(n, c.kv_heads, D)
            v_cache[li, pos:pos + n] = f16_array(v).reshape(n, c.kv_heads, D)
            qs = pround((qr * np.float32(1.0 / np.sqrt(D))).astype(np.float32))
            att = _attention(qs, k_cache[li], v_cache[li], pos, c.heads, c.kv_heads, D, pround, cu_count)
            h = (h + _linear(att, L.mats["o"], None, w, xround)).astype(np.float32)
            g = _projection(h, L.post_attention_norm, c.rms_eps, L.mats["gate"], None, w, xround, fold_pair)
            u = _projection(h, L.post_attention_norm, c.rms_eps, L.mats["up"], None, w, xround, fold_pair)
            g32 = g.astype(np.float32)
            a = (g32 / (np.float32(1.0) + np.exp(-g32)) * u.astype(np.float32)).astype(np.float32)
            h = (h + _linear(a, L.mats["down"], None, w, xround)).astype(np.float32)
    xf = rmsnorm(h[-1], model.final_norm, 1, H, c.rms_eps)
    return gemv_threads(xf, model.embedding, None, _threads())
