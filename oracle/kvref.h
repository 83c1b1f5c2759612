/*
 * kvref — CPU restatement of the reference engine's INT8 KV-cache semantics.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker for the HIP path:
 * only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load it.
 * The product (libbootstrap_hip.so and the bootstrap_hip package) never links,
 * imports or calls it, and has no CPU fallback.
 *
 * Every function cites the reference file:line it follows (paths relative to
 * the reference checkout). The reference itself (C#/.NET + Metal) cannot be
 * built or run on Linux, so it is restated here, not compiled.
 *
 * Pinning (what checks each function independently of its own formula):
 *   kvref_value_index      closed form + brute-force bijection over pages (tests)
 *   kvref_quantize/_store  bit-exact agreement with an independent NumPy float32
 *                          implementation; special cases (zero vector, amax
 *                          element -> +-127, exact .5 ties to even, -0.0, never -128);
 *                          invariant |c*s - x| <= s/2 (+1 ulp)
 *   kvref_half_bits        NumPy float16 RNE conversion, exhaustive over test ranges
 *   kvref_bf16_round       bit-level RNE definition vs NumPy (tests)
 *   kvref_rotate_f64       closed forms: position 0 is identity, |rotated pair| norm
 *                          preserved, d >= 64 passthrough, angle of j=0 equals position
 *   kvref_attention_f64    brute force vs an independent NumPy float64 softmax on
 *                          small shapes; one key -> v*sigmoid(g); equal scores ->
 *                          mean of v; equal queries -> equal outputs across heads
 *   kvref_attention_fp16kv_f64  an independent NumPy float64 softmax over FP16-decoded K/V
 *                          on small shapes; one key -> v*sigmoid(g); equal keys -> mean of
 *                          v; equal queries -> equal outputs across the heads of a group
 *   kvref_attention_online_emulate  p_mode 2 (no operand rounding) equals
 *                          kvref_attention_f64 to FP32 rounding, for 1-key and multi-tile
 *                          histories (the tile recurrence: maxima, decays, denominators);
 *                          one key -> exactly round(vs)*code*sigmoid(g) in each p_mode (the
 *                          operand rounding and where vs_ref enters); the BF16 and FP16
 *                          roundings themselves are pinned by NumPy/torch (kvref_half_bits,
 *                          kvref_bf16_round)
 *   kvref_fill_hash        reproduces the integer hash generator; known values
 *                          computed from the formula in Python integers (tests)
 */
#ifndef KVREF_H
#define KVREF_H
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

/* V byte offset inside the page-transposed INT8 V cache.
 * kernels.metal:126-128 (int8_value_index), Int8KvTests.cs:10 (ValueIndex). */
uint64_t kvref_value_index(uint32_t vector, uint32_t dimension);

/* Bytes of the INT8 V buffer for `length` tokens (whole 256-token pages).
 * Int8KvTests.cs:11 (ValueBytes), QwenEngine.cs:23 (Int8ValueCapacity). */
uint64_t kvref_value_bytes(uint32_t length);

/* Symmetric INT8 quantization of one 256-value vector.
 * kernels.metal:129-141 (store_kv_int8) and its C# twin Int8KvTests.cs:116-118:
 *   amax = max|x|; scale = amax/127 (fp32 RN); codes = clamp(rint(x*(127/amax)),-127,127),
 *   or code 0 and scale 0 when amax == 0. */
void kvref_quantize(const float *x, int8_t *codes, float *scale);

/* Append `rows` tokens of FP32 K and V ([rows][2][256]) at position `pos`:
 * vector (pos+row)*2+h; K codes token-major at vector*256+d, V codes at
 * kvref_value_index(vector,d), scales at ks/vs[vector].
 * kernels.metal:142-146 (batch_rope_int8 store half) with :129-141. */
void kvref_store(const float *k, const float *v, int rows, int pos,
                 int8_t *kc, int8_t *vc, float *ks, float *vs);

/* kvref_store with the rows split into contiguous blocks over `threads` POSIX threads
 * (each token's bytes are written by exactly one thread; same bytes as kvref_store). */
void kvref_store_mt(const float *k, const float *v, int rows, int pos,
                    int8_t *kc, int8_t *vc, float *ks, float *vs, int threads);

/* FP64 partial RoPE (theta = 1e7, dims 0..63 rotate in pairs j, j+32).
 * Int8KvTests.cs:13-18, KvStorageTests.cs:44-49; GPU form kernels.metal:122-125. */
double kvref_rotate_f64(const float *x, int d, int position);

/* float -> IEEE binary16 bits, round-to-nearest-even (C# (Half) cast,
 * Metal half(), used by kernels.metal:1276-1281 and Int8KvTests.cs:136). */
uint16_t kvref_half_bits(float f);
float kvref_half_to_float(uint16_t h);
/* float -> bfloat16 (RNE) -> float (Metal bfloat(), kernels.metal:1427). */
float kvref_bf16_round(float f);

/* FP32 [rows][16][256] query -> grouped FP16 [(h/G*rows+row)*G+h%G][256].
 * kernels.metal:1276-1281 (attention_query_grouped_half). */
void kvref_query_grouped_half(const float *x, int rows, int group, uint16_t *y);

/* FP64 causal GQA attention over the dequantized INT8 cache.
 * Int8KvTests.cs:130-157: logits[t] = q*code*ks[t*2+h/8]/16 with q optionally
 * FP16-rounded (prefill, Int8KvTests.cs:136) or FP32 (decode/verify,
 * kernels.metal:147-156); softmax in FP64; out = sum(p*vcode*vs)/(1+exp(-gate)).
 * Row r attends t <= pos + r. `bound` (nullable) receives
 * sum|p*vcode*vs|/(1+exp(-gate)), the reference's BF16 error scale
 * (Int8KvTests.cs:148,156). Work is split over `threads` POSIX threads. */
void kvref_attention_f64(const float *q, int round_q_half,
                         const int8_t *kc, const int8_t *vc,
                         const float *ks, const float *vs, const float *gate,
                         int rows, int pos, double *out, double *bound, int threads);

/* Same, over an FP16 K/V cache (token-major [t][2][256] half bits), the FP16
 * control storage (kernels.metal:16-21, 1356-1365; Int8KvTests.cs:138,149). */
void kvref_attention_fp16kv_f64(const float *q, int round_q_half,
                                const uint16_t *kh, const uint16_t *vh, const float *gate,
                                int rows, int pos, double *out, int threads);

/* The reference's tuned online INT8 prefill (kernels.metal:1378-1457) evaluated with its
 * roundings, one (row, head) at a time: FP16 Q, FP32 scores scaled by (1/16) and ks, 256-key
 * tiles (`tile_keys`) with a running FP32 maximum and denominator, probability operands
 * P = bfloat(e * vs) against BF16 x INT8 products, FP32 output. p_mode 0: that BF16 operand
 * (the reference); 1: FP16(e * vs / vs_ref), vs_ref = the largest V scale of the attended
 * keys, multiplied back at the end (this build's kernels); 2: no operand rounding. FP32 out
 * [rows][16][256]. Used to show what the operand rounding alone costs against FP64. */
void kvref_attention_online_emulate(const float *q, const int8_t *kc, const int8_t *vc,
                                    const float *ks, const float *vs, const float *gate,
                                    int rows, int pos, int tile_keys, int p_mode,
                                    float *out, int threads);

/* Deterministic integer-hash fill. FastAttentionTests.cs:111-119 (Fill). */
void kvref_fill_hash(float *out, int64_t count, uint32_t seed, float scale);

/* Raw splitmix64 stream (Steele, Lea, Flood 2014; Vigna's splitmix64.c): state += golden
 * gamma, then the two xor-shift-multiply rounds. Pinned by the published outputs for seed
 * 1234567. */
void kvref_splitmix64(uint64_t seed, uint64_t *out, int64_t count);
/* splitmix64 -> uniform (0,1) -> Box-Muller N(0,1), as float. */
void kvref_normal(float *out, int64_t count, uint64_t seed);
/* Student-t nu=4: z / sqrt(chi2_4 / 4), five normals per sample. */
void kvref_student_t4(float *out, int64_t count, uint64_t seed);

#ifdef __cplusplus
}
#endif
#endif
