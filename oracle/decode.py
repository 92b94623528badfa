"""CPU restatement of one decode step of the reference's model (test infrastructure only).

Composes the reference's CPU operators in decode order (graph_decode.ts:246-385 wires them;
test/reference/ops.ts defines them): embed (ops.ts:222-233, int8 dequantization
embedding_variants.ts:56-63), rmsNorm (:30-51), the quantized linears as linearQ4
(quant.ts:95-111, float64 sums, f32 results, via eo_gemv_threads), rope (:87-114),
attentionScores / softmaxRows / attentionApply for one query row (:130-205), siluMul
(:207-216), add (:218-220) and argmax (:237-244). Activations are stored as f32 between
operators, as the reference's Float32Arrays are; the KV cache holds f16-rounded rows when
`cache="f16"` (the reference's f16 cache variant, cache_variants.ts:147-305) and exact f32 rows
when `cache="f32"`.

Pinning: every operator it composes is pinned on its own (tests/test_oracle.py); `attention`
is pinned by closed forms in tests/test_decode_oracle.py (one position returns its value row,
equal keys average the values, a dominant score selects its row, GQA grouping).
The model is duck-typed: any object with the fields of enargeia_amd.model.HostModel.
"""

from __future__ import annotations

import os

import numpy as np

from . import gemv_threads, rmsnorm, rope


def _threads() -> int:
    try:
        return max(1, min(16, len(os.sched_getaffinity(0))))
    except AttributeError:
        return max(1, min(16, os.cpu_count() or 1))


def f16_array(a: np.ndarray) -> np.ndarray:
    """Round f32 values to binary16 and back (round to nearest even, numpy's conversion)."""
    with np.errstate(over="ignore"):  # beyond 65504 rounds to inf, as binary16 does
        return np.asarray(a, np.float32).astype(np.float16).astype(np.float32)


def attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, heads: int, kv_heads: int, head_dim: int) -> np.ndarray:
    """One decode row of ops.ts:130-205. q [heads*head_dim]; k, v [length][kv_heads][head_dim];
    returns f32 [heads*head_dim]. Scores scaled by 1/sqrt(head_dim), softmax max-subtracted, in
    float64."""
    group = heads // kv_heads
    qh = np.asarray(q, np.float64).reshape(heads, head_dim)
    kk = np.asarray(k, np.float64)
    vv = np.asarray(v, np.float64)
    out = np.empty((heads, head_dim), np.float64)
    scale = 1.0 / np.sqrt(head_dim)
    for h in range(heads):
        kv = h // group
        s = kk[:, kv, :] @ qh[h] * scale
        w = np.exp(s - s.max())
        w /= w.sum()
        out[h] = w @ vv[:, kv, :]
    return out.reshape(-1).astype(np.float32)


def prefill_attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, k_cache: np.ndarray, v_cache: np.ndarray,
                      begin: int, heads: int, kv_heads: int, head_dim: int, theta: float, cache: str = "f16"):
    """The reference's chunked prefill for one layer (graph.ts:411-459): RoPE on the chunk's q
    and k rows at positions begin + i (ops.ts:87-114), k and v written into the caches (f16
    rows for the f16 cache variant, the f32 rows themselves for `cache="f32"`,
    cache_variants.ts:21-40), then per query row i the causal attention over cache rows
    [0, begin + i] (attn_scores, softmax, attn_apply; cache_variants.ts:81-145), in float64.
    q [n][heads*D], k / v [n][kv_heads*D]; the caches [context][kv_heads][D] (f32 arrays) are
    updated in place. Returns (q_rope scaled by 1/sqrt(D), out [n][heads*D])."""
    n = q.shape[0]
    keep = f16_array if cache == "f16" else (lambda a: np.asarray(a, np.float32))
    qr = np.stack([rope(q[i], 1, heads, head_dim, theta, begin + i) for i in range(n)])
    kr = np.stack([rope(k[i], 1, kv_heads, head_dim, theta, begin + i) for i in range(n)])
    k_cache[begin:begin + n] = keep(kr).reshape(n, kv_heads, head_dim)
    v_cache[begin:begin + n] = keep(v).reshape(n, kv_heads, head_dim)
    out = np.stack([attention(qr[i], k_cache[:begin + i + 1], v_cache[:begin + i + 1], heads, kv_heads, head_dim)
                    for i in range(n)])
    return (qr * np.float32(1.0 / np.sqrt(head_dim))).astype(np.float32), out


def dense_values(q, begin: int = 0, end: int | None = None) -> np.ndarray:
    """Rows [begin, end) of an f16 (bits 16) or f32 (bits 32) table as f32 [rows][cols]
    (embedding_variants.ts:66-73: unpack2x16float takes element 2j from a word's low half)."""
    end = q.rows if end is None else end
    per = 32 // q.bits
    w = np.asarray(q.packed[begin * q.cols // per:end * q.cols // per], np.uint32)
    if q.bits == 32:
        return w.view(np.float32).reshape(end - begin, q.cols).copy()
    halves = np.stack([w & np.uint32(0xFFFF), w >> np.uint32(16)], axis=1).reshape(-1).astype(np.uint16)
    return halves.view(np.float16).astype(np.float32).reshape(end - begin, q.cols)


def dense_head(x: np.ndarray, q, rows_per_block: int = 8192) -> np.ndarray:
    """lm_head_f16 / lm_head_f32 (embedding_variants.ts:135-180): out[n] = sum_k table[n][k] x[k],
    summed in float64, f32 results (the table taken a block of rows at a time)."""
    x64 = np.asarray(x, np.float64)
    out = np.empty(q.rows, np.float32)
    for r0 in range(0, q.rows, rows_per_block):
        r1 = min(q.rows, r0 + rows_per_block)
        out[r0:r1] = (dense_values(q, r0, r1).astype(np.float64) @ x64).astype(np.float32)
    return out


def dequant_row(q, row: int) -> np.ndarray:
    """One row of a quantized table as f32 (embed, ops.ts:222-233, with the gather's dequant,
    embedding_variants.ts:56-63 / embed_gather_q4.wgsl): value = (code - zero) * scale per block
    for the offset encoding, code * scale with two's-complement codes for the signed one. Nibble
    n of a word is element 8w + n (byte b of a word is element 4w + b for int8). An f16 / f32
    table's row as it is (dense_values)."""
    if q.bits in (16, 32):
        return dense_values(q, row, row + 1)[0]
    per = 32 // q.bits
    mask = (1 << q.bits) - 1
    words = np.asarray(q.packed[row * q.cols // per:(row + 1) * q.cols // per], np.uint32)
    shifts = np.arange(per, dtype=np.uint32) * q.bits
    codes = ((words[:, None] >> shifts) & mask).reshape(-1).astype(np.int64)
    bpr = q.cols // q.block_size
    blocks = np.arange(row * bpr, (row + 1) * bpr)
    scales = np.asarray(q.scales, np.float32)[blocks]
    if q.zeros is None:  # signed: two's complement
        codes = np.where(codes >= (1 << (q.bits - 1)), codes - (1 << q.bits), codes)
        zero = np.zeros(bpr, np.int64)
    else:
        zw = np.asarray(q.zeros, np.uint32)[blocks // per]
        zero = ((zw >> ((blocks % per) * q.bits).astype(np.uint32)) & mask).astype(np.int64)
    vals = (codes.reshape(bpr, q.block_size) - zero[:, None]).astype(np.float32) * scales[:, None]
    return vals.reshape(-1).astype(np.float32)


def silu_mul(g: np.ndarray, u: np.ndarray) -> np.ndarray:
    g64 = np.asarray(g, np.float64)
    return (g64 / (1.0 + np.exp(-g64)) * np.asarray(u, np.float64)).astype(np.float32)


class OracleDecoder:
    """The model's decode step on the CPU, with its own KV cache."""

    def __init__(self, model, max_context: int | None = None, cache: str = "f16", threads: int | None = None):
        self.m = model
        c = model.cfg
        self.max_context = max_context or c.max_context
        self.cache = cache
        self.threads = threads or _threads()
        shape = (c.layers, self.max_context, c.kv_heads, c.head_dim)
        self.k = np.zeros(shape, np.float32)
        self.v = np.zeros(shape, np.float32)

    def embed(self, token: int) -> np.ndarray:
        return dequant_row(self.m.embedding, token)

    def linear(self, x: np.ndarray, q, bias=None) -> np.ndarray:
        return gemv_threads(x, q, bias, self.threads)

    def step(self, token: int, position: int) -> np.ndarray:
        """Logits (f32 [vocab]) of the token at `position`; appends its K/V to the cache."""
        c = self.m.cfg
        h = self.embed(token)
        for li, L in enumerate(self.m.layers):
            xn = rmsnorm(h, L.input_norm, 1, c.hidden, c.rms_eps)
            q = self.linear(xn, L.mats["q"], L.biases["q"])
            k = self.linear(xn, L.mats["k"], L.biases["k"])
            v = self.linear(xn, L.mats["v"], L.biases["v"])
            q = rope(q, 1, c.heads, c.head_dim, c.rope_theta, position)
            k = rope(k, 1, c.kv_heads, c.head_dim, c.rope_theta, position)
            kr = k.reshape(c.kv_heads, c.head_dim)
            vr = v.reshape(c.kv_heads, c.head_dim)
            self.k[li, position] = f16_array(kr) if self.cache == "f16" else kr
            self.v[li, position] = f16_array(vr) if self.cache == "f16" else vr
            attn = attention(q, self.k[li, :position + 1], self.v[li, :position + 1], c.heads, c.kv_heads,
                             c.head_dim)
            h = (h + self.linear(attn, L.mats["o"])).astype(np.float32)
            xn = rmsnorm(h, L.post_attention_norm, 1, c.hidden, c.rms_eps)
            a = silu_mul(self.linear(xn, L.mats["gate"]), self.linear(xn, L.mats["up"]))
            h = (h + self.linear(a, L.mats["down"])).astype(np.float32)
        xf = rmsnorm(h, self.m.final_norm, 1, c.hidden, c.rms_eps)
        if self.m.embedding.bits in (16, 32):  # an f16 / f32 tied table
            return dense_head(xf, self.m.embedding)
        return self.linear(xf, self.m.embedding)
