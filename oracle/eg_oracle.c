/*
 * eg_oracle.c — CPU restatement of the reference's quantized-projection semantics.
 *
 * TEST INFRASTRUCTURE ONLY. This is the checker, never the thing measured as the product and
 * never shipped in the product path: the HIP library does not link it and fails loudly on its
 * own when its kernels are missing. Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg load it.
 *
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off, no fast-math, so f32 statements stay
 * f32 statements and float64 statements stay float64, as in the reference's JS and WGSL).
 *
 * How each function is pinned (tests/test_oracle.py holds every check named here):
 *   mulberry32 / randomFloats  — JS-semantics vectors written by tests/golden/gen_js_vectors.js
 *                                (an independent JS statement run under the image's Node, so
 *                                Math.imul / >>> / Float32Array rounding are JS's own).
 *   eo_quantize_q4_ref         — known answers from test/kernels/matmul_q4.test.ts:96-146
 *                                (constant 0.375 block exact; endpoints -1.25/2.5 exact; error
 *                                <= step/2; blocks beat per-tensor) and JS-semantics vectors.
 *   eo_quantize_blocks_n       — closed forms: min -> code 0 and max -> code levels, error <=
 *                                scale/2, degenerate blocks (DECISIONS.md:522-530), ties-to-even
 *                                vs half-up on constructed halfway inputs.
 *   eo_quantize_sym            — closed forms: absmax element -> +-qmax exactly, |error| <=
 *                                scale/2, zero group -> scale 1 and code 0.
 *   eo_dequant                 — brute force over all 16 nibbles x 16 zeros and all 256 int8
 *                                codes in both encodings; word 0x76543210 -> elements 0..7.
 *   eo_linear_q                — x=1, W=0.5 => 0.5*K at outOffset with index 0 untouched
 *                                (matmul_q4.test.ts:181-195); agreement with numpy float64
 *                                matmul over the dequantized matrix; linearity in x.
 *   eo_linear_q_bf16           — equals eo_linear_q on inputs that are exactly bf16; bf16/f16
 *                                rounding checked against numpy/torch conversions.
 *   eo_argmax(_wgsl)           — forward_ops.test.ts:397-446 (seed 101, logits[123456]=99 ->
 *                                123456; tie at 100 and 900 -> 100) and numpy.argmax.
 *   eo_sample                  — the reference holds no CPU sampler and no sampled vectors:
 *                                pinned by properties only — T=0 equals argmax,
 *                                T=0.01/topP=1 equals greedy, kept mass >= topP, the draw is the
 *                                first ascending-id crossing, penalty set/sign rule against a
 *                                brute-force restatement, and an independent float64 nucleus
 *                                computation that must agree away from boundaries.
 *   eo_rmsnorm / eo_rope       — closed forms (mean-of-squares vs sum; position 0 unrotated;
 *                                half-rotation pairing i <-> i+headDim/2; norm preservation).
 */
#include "eg_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ---------------------------------------------------------------------------------------- */
/* RNG                                                                                       */
/* ---------------------------------------------------------------------------------------- */

/* test/reference/rng.ts:2-10. JS: s = (s + 0x6d2b79f5) >>> 0; t = Math.imul(s ^ s>>>15, 1|s);
 * t = (t + Math.imul(t ^ t>>>7, 61|t)) ^ t; return ((t ^ t>>>14) >>> 0) / 2^32.
 * All of it is exact in uint32 modular arithmetic (ToInt32 of the sum is the low 32 bits). */
void eo_mulberry32_init(eo_mulberry32* r, uint32_t seed) { r->s = seed; }

double eo_mulberry32_next(eo_mulberry32* r) {
  r->s += 0x6d2b79f5u;
  uint32_t s = r->s;
  uint32_t t = (s ^ (s >> 15)) * (1u | s);
  t = (t + (t ^ (t >> 7)) * (61u | t)) ^ t;
  return (double)(t ^ (t >> 14)) / 4294967296.0;
}

/* test/reference/rng.ts:13-18 */
void eo_random_floats(float* out, size_t count, uint32_t seed) {
  eo_mulberry32 r;
  eo_mulberry32_init(&r, seed);
  for (size_t i = 0; i < count; i++) out[i] = (float)(eo_mulberry32_next(&r) - 0.5);
}

void eo_normal_floats(float* out, size_t count, uint32_t seed, double sigma) {
  eo_mulberry32 r;
  eo_mulberry32_init(&r, seed);
  const double two_pi = 6.283185307179586476925286766559;
  for (size_t i = 0; i < count; i++) {
    double u1 = eo_mulberry32_next(&r);
    double u2 = eo_mulberry32_next(&r);
    double z = sqrt(-2.0 * log(1.0 - u1)) * cos(two_pi * u2);
    out[i] = (float)(z * sigma);
  }
}

void eo_random_ids(uint32_t* out, size_t count, uint32_t seed, uint32_t bound) {
  eo_mulberry32 r;
  eo_mulberry32_init(&r, seed);
  for (size_t i = 0; i < count; i++) {
    uint32_t v = (uint32_t)floor(eo_mulberry32_next(&r) * (double)bound);
    out[i] = v < bound ? v : bound - 1;
  }
}

/* ---------------------------------------------------------------------------------------- */
/* Quantizers                                                                                */
/* ---------------------------------------------------------------------------------------- */

/* JS Math.round: nearest integer, halfway cases toward +infinity. floor(x + 0.5) is wrong for
 * 0.49999999999999994, so the fraction is compared instead (x - floor(x) is exact here). */
static double js_round(double x) {
  if (!isfinite(x)) return x;
  double r = floor(x);
  if (x - r >= 0.5) r += 1.0;
  return r;
}

static double clampd(double v, double lo, double hi) { return v < lo ? lo : (v > hi ? hi : v); }

/* test/reference/quant.ts:24-74. Float64 throughout; `scale` stays float64 for the codes and
 * is rounded to f32 only where it is stored (quant.ts:42 scales[b] = scale). */
int eo_quantize_q4_ref(const float* values, int rows, int cols, int block_size,
                       uint32_t* packed, float* scales, uint32_t* zeros) {
  if (block_size <= 0 || cols % block_size != 0) return -1;
  const size_t elements = (size_t)rows * (size_t)cols;
  if (elements % 8 != 0) return -1;
  const size_t blocks = elements / (size_t)block_size;
  uint32_t* q = (uint32_t*)malloc(elements * sizeof(uint32_t));
  uint32_t* zv = (uint32_t*)malloc(blocks * sizeof(uint32_t));
  if (!q || !zv) { free(q); free(zv); return -2; }
  for (size_t b = 0; b < blocks; b++) {
    double lo = INFINITY, hi = -INFINITY;
    for (int i = 0; i < block_size; i++) {
      double v = values[b * block_size + i];
      if (v < lo) lo = v;
      if (v > hi) hi = v;
    }
    double scale = (hi - lo) / 15.0;
    if (!(scale > 0)) scale = hi != 0 ? fabs(hi) / 15.0 : 1.0;
    double zero = fmin(15.0, fmax(0.0, js_round(-lo / scale)));
    scales[b] = (float)scale;
    zv[b] = (uint32_t)zero;
    for (int i = 0; i < block_size; i++) {
      double code = js_round((double)values[b * block_size + i] / scale + zero);
      q[b * block_size + i] = (uint32_t)fmin(15.0, fmax(0.0, code));
    }
  }
  for (size_t w = 0; w < elements / 8; w++) {
    uint32_t word = 0;
    for (int n = 0; n < 8; n++) word |= q[w * 8 + n] << (n * 4);
    packed[w] = word;
  }
  for (size_t w = 0; w < (blocks + 7) / 8; w++) {
    uint32_t word = 0;
    for (int n = 0; n < 8; n++) {
      size_t b = w * 8 + n;
      if (b < blocks) word |= zv[b] << (n * 4);
    }
    zeros[w] = word;
  }
  free(q);
  free(zv);
  return 0;
}

/* tools/quantize.py:74-103. numpy float32 semantics: lo/hi/scale/zero in f32 with rint
 * (ties-to-even); the code is rint of (f32 quotient widened to float64) + int64 zero, because
 * numpy promotes float32 + int64 to float64 (quantize.py:93). */
int eo_quantize_blocks_n(const float* values, int rows, int cols, int block_size, int bits,
                         uint32_t* packed, float* scales, uint32_t* zeros) {
  if ((bits != 4 && bits != 8) || block_size <= 0 || cols % block_size != 0) return -1;
  const int levels = (1 << bits) - 1;
  const int per_word = 32 / bits;
  const size_t elements = (size_t)rows * (size_t)cols;
  if (elements % (size_t)per_word != 0) return -1;
  const size_t blocks = elements / (size_t)block_size;
  memset(packed, 0, elements / per_word * sizeof(uint32_t));
  memset(zeros, 0, (blocks + per_word - 1) / per_word * sizeof(uint32_t));
  for (size_t b = 0; b < blocks; b++) {
    float lo = INFINITY, hi = -INFINITY;
    for (int i = 0; i < block_size; i++) {
      float v = values[b * block_size + i];
      lo = v < lo ? v : lo;
      hi = v > hi ? v : hi;
    }
    float scale = (hi - lo) / (float)levels;
    if (scale <= 0.0f) scale = hi != 0.0f ? fabsf(hi) / (float)levels : 1.0f;
    float zf = rintf(-lo / scale);
    int64_t zero = (int64_t)(zf < 0.0f ? 0.0f : (zf > (float)levels ? (float)levels : zf));
    scales[b] = scale;
    zeros[b / per_word] |= (uint32_t)zero << (bits * (b % per_word));
    for (int i = 0; i < block_size; i++) {
      size_t e = b * block_size + i;
      float quotient = values[e] / scale;
      double code = clampd(rint((double)quotient + (double)zero), 0.0, (double)levels);
      packed[e / per_word] |= (uint32_t)code << (bits * (e % per_word));
    }
  }
  return 0;
}

int eo_quantize_sym(const float* values, int rows, int cols, int block_size, int bits,
                    uint32_t* packed, float* scales) {
  if ((bits != 4 && bits != 8) || block_size <= 0 || cols % block_size != 0) return -1;
  const int qmax = bits == 4 ? 7 : 127;
  const int per_word = 32 / bits;
  const uint32_t mask = bits == 4 ? 0xFu : 0xFFu;
  const size_t elements = (size_t)rows * (size_t)cols;
  if (elements % (size_t)per_word != 0) return -1;
  const size_t blocks = elements / (size_t)block_size;
  memset(packed, 0, elements / per_word * sizeof(uint32_t));
  for (size_t b = 0; b < blocks; b++) {
    float absmax = 0.0f;
    for (int i = 0; i < block_size; i++) {
      float a = fabsf(values[b * block_size + i]);
      absmax = a > absmax ? a : absmax;
    }
    float scale = absmax > 0.0f ? absmax / (float)qmax : 1.0f;
    scales[b] = scale;
    for (int i = 0; i < block_size; i++) {
      size_t e = b * block_size + i;
      float code = rintf(values[e] / scale);
      code = code < (float)(-qmax - 1) ? (float)(-qmax - 1) : (code > (float)qmax ? (float)qmax : code);
      uint32_t bitsv = (uint32_t)(int32_t)code & mask;
      packed[e / per_word] |= bitsv << (bits * (e % per_word));
    }
  }
  return 0;
}

/* ---------------------------------------------------------------------------------------- */
/* Dequant / GEMV                                                                            */
/* ---------------------------------------------------------------------------------------- */

static inline int32_t code_at(const uint32_t* packed, int bits, size_t e) {
  const int per_word = 32 / bits;
  const uint32_t mask = bits == 4 ? 0xFu : 0xFFu;
  return (int32_t)((packed[e / per_word] >> (bits * (e % per_word))) & mask);
}

/* quant.ts:77-84 / matmul_q4_decode.wgsl:73-79 (int4), embedding_variants.ts:56-63 (int8).
 * The value is (code - zero) * scale in float64, as the JS reference computes it. */
double eo_dequant(const uint32_t* packed, const float* scales, const uint32_t* zeros, int bits,
                  int encoding, int cols, int block_size, int row, int col) {
  const size_t flat = (size_t)row * cols + col;
  const size_t block = (size_t)row * (cols / block_size) + col / block_size;
  int32_t code = code_at(packed, bits, flat);
  int32_t zero;
  if (encoding == EO_ENC_OFFSET_ZEROS) {
    zero = code_at(zeros, bits, block);
  } else {
    const int32_t half = 1 << (bits - 1);
    code = code >= half ? code - (1 << bits) : code; /* sign-extend the two's-complement code */
    zero = 0;
  }
  return (double)(code - zero) * (double)scales[block];
}

/* test/reference/quant.ts:95-111 */
void eo_linear_q(const float* x, int m, int k, int n, const uint32_t* packed, const float* scales,
                 const uint32_t* zeros, int block_size, int bits, int encoding, const float* bias,
                 float* out, int out_stride, int out_offset) {
  for (int row = 0; row < m; row++) {
    for (int col = 0; col < n; col++) {
      double acc = bias ? (double)bias[col] : 0.0;
      for (int i = 0; i < k; i++)
        acc += (double)x[(size_t)row * k + i] *
               eo_dequant(packed, scales, zeros, bits, encoding, k, block_size, col, i);
      out[(size_t)row * out_stride + col + out_offset] = (float)acc;
    }
  }
}

float eo_bf16_round(float v) {
  uint32_t u;
  memcpy(&u, &v, 4);
  if ((u & 0x7F800000u) == 0x7F800000u) { /* inf / nan: truncate, keep nan quiet */
    u &= 0xFFFF0000u;
    if (isnan(v)) u |= 0x00400000u;
  } else {
    u += 0x7FFFu + ((u >> 16) & 1u);
    u &= 0xFFFF0000u;
  }
  float r;
  memcpy(&r, &u, 4);
  return r;
}

float eo_f16_round(float v) {
  /* Round to the nearest IEEE binary16 value (ties to even), returned widened to f32. */
  if (!isfinite(v)) return v;
  float a = fabsf(v);
  if (a >= 65520.0f) return copysignf(INFINITY, v);
  if (a < 6.103515625e-05f) { /* subnormal range: quantum 2^-24 */
    float q = rintf(a / 5.9604644775390625e-08f) * 5.9604644775390625e-08f;
    return copysignf(q, v);
  }
  int e;
  frexpf(a, &e);                       /* a = f * 2^e, f in [0.5, 1) */
  float quantum = ldexpf(1.0f, e - 11); /* 11 significant bits */
  return copysignf(rintf(a / quantum) * quantum, v);
}

void eo_linear_q_bf16(const float* x, int m, int k, int n, const uint32_t* packed,
                      const float* scales, const uint32_t* zeros, int block_size, int bits,
                      int encoding, const float* bias, float* out, int out_stride, int out_offset) {
  for (int row = 0; row < m; row++) {
    for (int col = 0; col < n; col++) {
      double acc = 0.0;
      for (int i = 0; i < k; i++) {
        /* The device computes (code - zero) * scale in f32 before rounding to bf16. */
        float w = (float)eo_dequant(packed, scales, zeros, bits, encoding, k, block_size, col, i);
        acc += (double)eo_bf16_round(x[(size_t)row * k + i]) * (double)eo_bf16_round(w);
      }
      if (bias) acc += (double)bias[col];
      out[(size_t)row * out_stride + col + out_offset] = (float)acc;
    }
  }
}

/* ---------------------------------------------------------------------------------------- */
/* argmax / sampling                                                                         */
/* ---------------------------------------------------------------------------------------- */

/* test/reference/ops.ts:237-244 */
uint32_t eo_argmax(const float* x, size_t n) {
  size_t best = 0;
  for (size_t i = 1; i < n; i++)
    if (x[i] > x[best]) best = i;
  return (uint32_t)best;
}

/* argmax.wgsl:28-66 */
uint32_t eo_argmax_wgsl(const float* x, size_t n) {
  enum { WG = 256 };
  float value[WG];
  uint32_t index[WG];
  for (int t = 0; t < WG; t++) {
    float v = -1.0e30f;
    uint32_t idx = 0;
    for (size_t i = t; i < n; i += WG)
      if (x[i] > v) { v = x[i]; idx = (uint32_t)i; }
    value[t] = v;
    index[t] = idx;
  }
  for (int stride = WG / 2; stride > 0; stride /= 2)
    for (int t = 0; t < stride; t++) {
      int o = t + stride;
      if (value[o] > value[t] || (value[o] == value[t] && index[o] < index[t])) {
        value[t] = value[o];
        index[t] = index[o];
      }
    }
  return index[0];
}

enum { SWG = 256, BISECTION_STEPS = 32 };

/* sample.wgsl:115-141: the 256-slot tree, strides 128..1. */
static float tree_sum(float* r) {
  for (int stride = SWG / 2; stride > 0; stride /= 2)
    for (int t = 0; t < stride; t++) r[t] = r[t] + r[t + stride];
  return r[0];
}

static void tree_argmax(float* r, uint32_t* idx) {
  for (int stride = SWG / 2; stride > 0; stride /= 2)
    for (int t = 0; t < stride; t++) {
      int o = t + stride;
      if (r[o] > r[t] || (r[o] == r[t] && idx[o] < idx[t])) {
        r[t] = r[o];
        idx[t] = idx[o];
      }
    }
}

/* sample.wgsl:67-74 */
static uint32_t chunk_begin(uint32_t tid, uint32_t vocab) {
  uint32_t per = (vocab + SWG - 1) / SWG;
  uint32_t b = tid * per;
  return b < vocab ? b : vocab;
}
static uint32_t chunk_end(uint32_t tid, uint32_t vocab) {
  uint32_t per = (vocab + SWG - 1) / SWG;
  uint32_t e = (tid + 1) * per;
  return e < vocab ? e : vocab;
}

/* p for one logit, exactly the expression sample.wgsl:248,268,288,311 evaluates. */
static inline float prob(float logit, float temperature, float mx, float sum) {
  return expf(logit / temperature - mx) / sum;
}

/* sample.wgsl:91-113 (applyRepetitionPenalty) through :332 (the draw and the fallback). */
uint32_t eo_sample(float* logits, uint32_t vocab, const uint32_t* history, uint32_t history_len,
                   float temperature, float top_p, float repetition_penalty, float random,
                   eo_sample_info* info) {
  eo_sample_info local;
  if (!info) info = &local;
  memset(info, 0, sizeof(*info));
  info->bisect_margin = INFINITY;
  info->threshold_gap = INFINITY;
  info->draw_margin = INFINITY;

  /* Penalty: each id's first occurrence applies it once; divide positives, multiply negatives. */
  if (repetition_penalty != 1.0f) {
    for (uint32_t h = 0; h < history_len; h++) {
      uint32_t id = history[h];
      int first = 1;
      for (uint32_t e = 0; e < h; e++)
        if (history[e] == id) { first = 0; break; }
      if (first && id < vocab) {
        float v = logits[id];
        logits[id] = v > 0.0f ? v / repetition_penalty : v * repetition_penalty;
      }
    }
  }

  float r[SWG];
  uint32_t ri[SWG];

  if (temperature <= 0.0f) { /* sample.wgsl:165-195 */
    for (uint32_t t = 0; t < SWG; t++) {
      float best = -1.0e30f;
      uint32_t bi = 0;
      for (uint32_t i = chunk_begin(t, vocab); i < chunk_end(t, vocab); i++)
        if (logits[i] > best) { best = logits[i]; bi = i; }
      r[t] = best;
      ri[t] = bi;
    }
    tree_argmax(r, ri);
    info->greedy = 1;
    info->token = ri[0];
    info->argmax = ri[0];
    return ri[0];
  }

  /* max / argmax of l/T: sample.wgsl:198-228 */
  for (uint32_t t = 0; t < SWG; t++) {
    uint32_t b = chunk_begin(t, vocab);
    float lm = -1.0e30f;
    uint32_t la = b;
    for (uint32_t i = b; i < chunk_end(t, vocab); i++) {
      float scaled = logits[i] / temperature;
      if (scaled > lm) { lm = scaled; la = i; }
    }
    r[t] = lm;
    ri[t] = la;
  }
  tree_argmax(r, ri);
  const float mx = r[0];
  const uint32_t amax = ri[0];

  /* sum of exp: sample.wgsl:230-236 */
  for (uint32_t t = 0; t < SWG; t++) {
    float s = 0.0f;
    for (uint32_t i = chunk_begin(t, vocab); i < chunk_end(t, vocab); i++)
      s = s + expf(logits[i] / temperature - mx);
    r[t] = s;
  }
  const float total = tree_sum(r);

  /* bisection: sample.wgsl:241-261 */
  float lo = 0.0f, hi = 1.0f;
  if (top_p < 1.0f) {
    for (int step = 0; step < BISECTION_STEPS; step++) {
      float mid = (lo + hi) * 0.5f;
      for (uint32_t t = 0; t < SWG; t++) {
        float m = 0.0f;
        for (uint32_t i = chunk_begin(t, vocab); i < chunk_end(t, vocab); i++) {
          float p = prob(logits[i], temperature, mx, total);
          if (p >= mid) m = m + p;
        }
        r[t] = m;
      }
      float mass = tree_sum(r);
      double margin = fabs((double)mass - (double)top_p);
      if (margin < info->bisect_margin) info->bisect_margin = margin;
      if (mass < top_p) hi = mid; else lo = mid;
    }
  }
  const float threshold = top_p < 1.0f ? lo : 0.0f;

  /* kept mass: sample.wgsl:266-279, and the per-chunk totals for the scan :286-306 */
  float mine[SWG];
  uint32_t kept_count = 0;
  float min_kept = INFINITY, max_excluded = -INFINITY;
  for (uint32_t t = 0; t < SWG; t++) {
    float s = 0.0f;
    for (uint32_t i = chunk_begin(t, vocab); i < chunk_end(t, vocab); i++) {
      float p = prob(logits[i], temperature, mx, total);
      if (p >= threshold) {
        s = s + p;
        kept_count++;
        if (p < min_kept) min_kept = p;
      } else if (p > max_excluded) {
        max_excluded = p;
      }
    }
    r[t] = s;
    mine[t] = s;
  }
  /* How far apart the kept set's smallest p and the largest excluded p are: the kept set
   * is robust to rounding differences in p and in the masses only when this gap is clear. */
  if (top_p < 1.0f && max_excluded > -INFINITY && min_kept < INFINITY)
    info->threshold_gap = ((double)min_kept - (double)max_excluded) / (double)min_kept;
  const float kept = tree_sum(r);
  const float target = random * (kept > 1.0e-20f ? kept : 1.0e-20f);

  /* exclusive serial scan, then each chunk's first crossing; lowest id wins :286-331 */
  float prefix[SWG];
  float running = 0.0f;
  for (uint32_t t = 0; t < SWG; t++) {
    prefix[t] = running;
    running = running + mine[t];
  }
  uint32_t chosen = 0xFFFFFFFFu;
  double draw_margin = INFINITY;
  for (uint32_t t = 0; t < SWG && chosen == 0xFFFFFFFFu; t++) {
    float run = prefix[t];
    for (uint32_t i = chunk_begin(t, vocab); i < chunk_end(t, vocab); i++) {
      float p = prob(logits[i], temperature, mx, total);
      if (p >= threshold) {
        float before = run;
        run = run + p;
        if (run >= target) {
          chosen = i;
          double a = ((double)target - (double)before) / (double)kept;
          double b = ((double)run - (double)target) / (double)kept;
          draw_margin = fabs(a) < fabs(b) ? fabs(a) : fabs(b);
          break;
        }
      }
    }
  }
  info->greedy = 0;
  info->max_scaled = mx;
  info->argmax = amax;
  info->total = total;
  info->threshold = threshold;
  info->kept = kept;
  info->target = target;
  info->draw_margin = draw_margin;
  info->kept_count = kept_count;
  info->token = chosen == 0xFFFFFFFFu ? amax : chosen;
  return info->token;
}

/* ---------------------------------------------------------------------------------------- */
/* Decode-step reference ops                                                                 */
/* ---------------------------------------------------------------------------------------- */

/* test/reference/ops.ts:30-51 */
void eo_rmsnorm(const float* x, const float* w, float* out, int seq, int features, double eps) {
  for (int s = 0; s < seq; s++) {
    double sum = 0.0;
    for (int f = 0; f < features; f++) {
      double v = x[(size_t)s * features + f];
      sum += v * v;
    }
    double scale = 1.0 / sqrt(sum / features + eps);
    for (int f = 0; f < features; f++)
      out[(size_t)s * features + f] = (float)((double)x[(size_t)s * features + f] * scale * (double)w[f]);
  }
}

/* test/reference/ops.ts:87-114 (in place on x) */
void eo_rope(float* x, int seq, int heads, int head_dim, double theta, int position_offset) {
  const int half = head_dim / 2;
  for (int s = 0; s < seq; s++) {
    double position = (double)(s + position_offset);
    for (int h = 0; h < heads; h++) {
      size_t base = ((size_t)s * heads + h) * head_dim;
      for (int i = 0; i < half; i++) {
        double freq = 1.0 / pow(theta, (2.0 * i) / head_dim);
        double angle = position * freq;
        double c = cos(angle), sn = sin(angle);
        double a = x[base + i], b = x[base + i + half];
        x[base + i] = (float)(a * c - b * sn);
        x[base + i + half] = (float)(b * c + a * sn);
      }
    }
  }
}

/* test/reference/ops.ts:207-209 */
float eo_silu(float v) { return (float)((double)v / (1.0 + exp(-(double)v))); }

/* ---------------------------------------------------------------------------------------- */
/* CPU baseline                                                                              */
/* ---------------------------------------------------------------------------------------- */

typedef struct {
  const float* x;
  int k, n0, n1;
  const uint32_t* packed;
  const float* scales;
  const uint32_t* zeros;
  int block_size, bits, encoding;
  const float* bias;
  float* out;
} gemv_job;

static void* gemv_worker(void* arg) {
  gemv_job* j = (gemv_job*)arg;
  for (int col = j->n0; col < j->n1; col++) {
    double acc = j->bias ? (double)j->bias[col] : 0.0;
    for (int i = 0; i < j->k; i++)
      acc += (double)j->x[i] * eo_dequant(j->packed, j->scales, j->zeros, j->bits, j->encoding,
                                          j->k, j->block_size, col, i);
    j->out[col] = (float)acc;
  }
  return NULL;
}

void eo_gemv_threads(const float* x, int k, int n, const uint32_t* packed, const float* scales,
                     const uint32_t* zeros, int block_size, int bits, int encoding,
                     const float* bias, float* out, int threads) {
  if (threads < 1) threads = 1;
  if (threads > 256) threads = 256;
  gemv_job jobs[256];
  pthread_t tids[256];
  for (int t = 0; t < threads; t++) {
    jobs[t] = (gemv_job){x, k, (int)((long)n * t / threads), (int)((long)n * (t + 1) / threads),
                         packed, scales, zeros, block_size, bits, encoding, bias, out};
  }
  if (threads == 1) {
    gemv_worker(&jobs[0]);
    return;
  }
  for (int t = 0; t < threads; t++) pthread_create(&tids[t], NULL, gemv_worker, &jobs[t]);
  for (int t = 0; t < threads; t++) pthread_join(tids[t], NULL);
}
