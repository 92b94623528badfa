/*
 * eg_oracle — CPU restatement of the Enargeia reference semantics for the quantized projection
 * hot path. TEST INFRASTRUCTURE ONLY: this library is the checker that the HIP path is compared
 * against. Nothing in the product (the HIP library, its C ABI, the Python or JS host mirrors)
 * links or calls it; only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg do.
 *
 * Every function cites the reference file:line it restates (paths relative to the reference
 * repository root). Numeric conventions follow the reference: the TypeScript CPU reference
 * computes in float64 (JS numbers) and stores into Float32Array; the WGSL kernels compute in f32.
 *
 * Parity pinning (what checks each function against something other than itself) is listed in
 * the header comment of eg_oracle.c.
 */
#ifndef EG_ORACLE_H
#define EG_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Quantized weight encodings (see include/enargeia_hip.h for the device-side contract). */
enum {
  EO_ENC_OFFSET_ZEROS = 0, /* unsigned code, explicit per-block zero-point stream (reference) */
  EO_ENC_SIGNED = 1,       /* two's-complement code, implicit zero         */
};

/* ---- RNG ------------------------------------------------------------------------------- */
/* mulberry32: test/reference/rng.ts:2-10, src/runtime/session.ts:75-83. Returns successive
 * doubles in [0,1) exactly as the JS closure does. */
typedef struct { uint32_t s; } eo_mulberry32;
void eo_mulberry32_init(eo_mulberry32* r, uint32_t seed);
double eo_mulberry32_next(eo_mulberry32* r);
/* randomFloats: test/reference/rng.ts:13-18 — Float32Array of (rand() - 0.5). */
void eo_random_floats(float* out, size_t count, uint32_t seed);
/* Normal(0, sigma) by Box-Muller over mulberry32 draws (this build's own synthetic generator,
 * used for the BASELINE configs): z = sqrt(-2 ln(1-u1)) * cos(2 pi u2), one value per pair. */
void eo_normal_floats(float* out, size_t count, uint32_t seed, double sigma);
/* Uniform integer ids in [0, bound) from mulberry32: floor(u * bound). */
void eo_random_ids(uint32_t* out, size_t count, uint32_t seed, uint32_t bound);

/* ---- quantizers -------------------------------------------------------------------------- */
/* Reference asymmetric int4: test/reference/quant.ts:24-74 (float64, Math.round half-up). */
int eo_quantize_q4_ref(const float* values, int rows, int cols, int block_size,
                       uint32_t* packed, float* scales, uint32_t* zeros);
/* Reference asymmetric int-n (4 or 8) as tools/quantize.py:74-103 writes it (float32, rint
 * ties-to-even). int8 is the shipped embedding format (quantize.py:135-149). */
int eo_quantize_blocks_n(const float* values, int rows, int cols, int block_size, int bits,
                         uint32_t* packed, float* scales, uint32_t* zeros);
/* BASELINE symmetric formats (configs 0-4): scale = absmax/qmax in f32 (1.0 for an all-zero
 * group), q = rint(v/scale) clamped to [-qmax-1, qmax], two's-complement, packed little-endian
 * (element 2j in the low nibble of byte j for int4; byte e&3 of word e>>2 for int8).
 * bits=4: qmax=7, group = block_size along K. bits=8: qmax=127, block_size = cols for per-row. */
int eo_quantize_sym(const float* values, int rows, int cols, int block_size, int bits,
                    uint32_t* packed, float* scales);

/* ---- dequant / GEMV ---------------------------------------------------------------------- */
/* One weight, by the shaders' indexing: quant.ts:77-84, matmul_q4_decode.wgsl:73-79,
 * embedding_variants.ts:56-63. zeros may be NULL for EO_ENC_SIGNED. */
double eo_dequant(const uint32_t* packed, const float* scales, const uint32_t* zeros, int bits,
                  int encoding, int cols, int block_size, int row, int col);
/* out[m,n] = sum_k x[m,k] * dequant(W)[n,k] + bias[n], float64 accumulate, f32 store:
 * test/reference/quant.ts:95-111 (linearQ4), generalised over bits/encoding.
 * Output row r is written at out[r*out_stride + col + out_offset] (matmul_q4_prefill.wgsl:154). */
void eo_linear_q(const float* x, int m, int k, int n, const uint32_t* packed, const float* scales,
                 const uint32_t* zeros, int block_size, int bits, int encoding, const float* bias,
                 float* out, int out_stride, int out_offset);
/* The bf16-MFMA prefill model: bf16(x) . bf16(dequant W), products exact, float64 accumulate,
 * plus bias, f32 store. bf16 rounding is round-to-nearest-even. */
void eo_linear_q_bf16(const float* x, int m, int k, int n, const uint32_t* packed,
                      const float* scales, const uint32_t* zeros, int block_size, int bits,
                      int encoding, const float* bias, float* out, int out_stride, int out_offset);
float eo_bf16_round(float v);
float eo_f16_round(float v);

/* ---- argmax / sampling ------------------------------------------------------------------- */
/* Lowest index of the maximum: test/reference/ops.ts:237-244. */
uint32_t eo_argmax(const float* x, size_t n);
/* argmax.wgsl:28-66: strided per-lane max from a -1e30 sentinel, ties to the lower index.
 * Differs from eo_argmax only for all-(<= -1e30) inputs. */
uint32_t eo_argmax_wgsl(const float* x, size_t n);

typedef struct {
  uint32_t token;
  int greedy;
  float max_scaled;      /* sharedMax */
  uint32_t argmax;       /* sharedArgmax */
  float total;           /* sharedSum */
  float threshold;       /* nucleus threshold after bisection (0 when topP >= 1) */
  float kept;            /* retained mass */
  float target;          /* random * max(kept, 1e-20) */
  /* Closest approach of a decision to its boundary: min over bisection steps of |mass - topP|;
   * (smallest kept p - largest excluded p) / smallest kept p; and the distance of the target
   * from the cumulative sums on either side of the chosen id, relative to the kept mass. */
  double bisect_margin;
  double threshold_gap;
  double draw_margin;
  uint32_t kept_count;
} eo_sample_info;

/* sample.wgsl:143-332 (with applyRepetitionPenalty :91-113, reductions :115-141, chunks
 * :67-74), in f32 with the same 256-lane chunking and tree-reduction order. `logits` is
 * modified in place by the penalty, as the kernel does. */
uint32_t eo_sample(float* logits, uint32_t vocab, const uint32_t* history, uint32_t history_len,
                   float temperature, float top_p, float repetition_penalty, float random,
                   eo_sample_info* info);

/* ---- decode-step reference ops (test/reference/ops.ts) ---------------------------------- */
void eo_rmsnorm(const float* x, const float* w, float* out, int seq, int features, double eps);
void eo_rope(float* x, int seq, int heads, int head_dim, double theta, int position_offset);
float eo_silu(float v);

/* ---- CPU baseline: the linearQ4 loop, timed --------------------------------------------- */
/* Same arithmetic as eo_linear_q for m=1, parallel over output rows with `threads` POSIX
 * threads (1 = the single-threaded reference loop). Returns nothing; writes out. */
void eo_gemv_threads(const float* x, int k, int n, const uint32_t* packed, const float* scales,
                     const uint32_t* zeros, int block_size, int bits, int encoding,
                     const float* bias, float* out, int threads);

#ifdef __cplusplus
}
#endif
#endif
