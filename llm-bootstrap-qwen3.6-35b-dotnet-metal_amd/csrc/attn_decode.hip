// Single-token (and 1-8 row verification) INT8 attention over the KV cache.
//
// Two entry points:
//   * the reference's three-kernel reader (kernels.metal:147-156,163-166):
//     batch_attention_scores_int8 -> attention_softmax -> batch_attention_values_int8,
//     FP32 scores in a caller buffer; serves serial decode and speculative
//     verification unchanged (QwenEngine.cs:161-165, Prefill.cs:280-285).
//   * attention_decode_int8: one fused split-K pass that streams the INT8 K/V
//     pages from HBM once, as whole K rows and whole 128-byte V page-row lines
//     staged through LDS. Scores run on INT8 MFMA straight from the K codes:
//     the FP32 query of each head is split into three INT8 parts,
//     q ~= s_q (q1 + q2 / 254 + q3 / 254^2) with s_q = max|q| / 127 (error
//     <= 6.1e-8 max|q| per element, below the FP32 reader's own summation error),
//     in two MFMAs whose 16 columns are 8 heads x {q1, q2} and 8 heads x q3. PV runs on FP16 MFMA
//     with V codes dequantized exactly in registers and the scaled
//     probabilities p*vs[t]/vs_ref (vs_ref = the largest V scale of the split, so
//     they lie in [0, 1]) split into FP16 hi + lo. Scales are applied to scores
//     and probabilities as the reference does (score = dot * ks[t] / 16,
//     P = p * vs[t]).
#include "common.h"
#include <type_traits>
#include "kvmath.h"
#include "mfma.h"

namespace boot {


namespace {

// ---------------------------------------------------------------- reference-compatible reader

// scores[(row*16+h)*K + t] = (q . code) * ks[t*2+h/8] * (1/16), -inf beyond row's causal end
// (kernels.metal:147-152), on INT8 MFMA (v_mfma_i32_16x16x64_i8). Each (row, head) query is split
// into three INT8 parts, q ~= s_q (q1 + q2 / 254 + q3 / 254^2) with s_q = max|q| / 127 (error
// <= 6.1e-8 max|q| per element), the dot products with the codes are exact integers, and their
// combination is FP32 per element: a row's scores do not depend on the rows it is dispatched
// with. Work-group (span = 256 or 512 tokens, KV group, kRows rows): the query operands of its rows
// in LDS (16 columns: 8 heads x {q1, q2}, and 8 heads x q3 twice), wave w takes the span's quarter
// w in pairs of 16-token tiles; each K operand (16 bytes of a token's row per lane) feeds 2 kRows
// MFMAs.
template <int kRows>
__global__ __launch_bounds__(256) void scores_int8_kernel(const float *__restrict__ q, const int8_t *__restrict__ k,
                                                          float *__restrict__ scores, const float *__restrict__ ks,
                                                          uint32_t rows, uint32_t K, uint32_t pos, uint32_t tiles,
                                                          uint32_t zs, uint32_t span) {
    typedef int v4i __attribute__((ext_vector_type(4)));
    __shared__ v4i qop[kRows][2][4][64];   // [row][set][64-dimension step][lane]
    __shared__ float qscale[kRows][8];
    // blocks are dealt to the XCDs round-robin by index: the row blocks of one (tile, group) pair
    // are 8 apart, on one XCD at about the same time, so that the K tile they share comes from HBM once
    const uint32_t xcd = blockIdx.x % 8, j = blockIdx.x / 8, pair = (j / zs) * 8 + xcd;
    if (pair >= 2 * tiles) return;   // padding of the grid to whole rounds of 8
    const uint32_t kt = pair / 2, g = pair % 2, r0 = (j % zs) * kRows;
    const uint32_t nr = min((uint32_t)kRows, rows - r0);
    const uint32_t length = min(pos + rows, K);   // the cache rows read (validated by the launcher)
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, n = lane & 15, qq = lane >> 4;
    // ---- query parts: thread T takes head T / 32, dimensions 8 (T % 32) .. + 7 of each row
    {
        const int h = tid >> 5, d0 = 8 * (tid & 31);
        auto code = [](float x) { return (uint32_t)(uint8_t)(int8_t)(int)fminf(fmaxf(x, -127.0f), 127.0f); };
#pragma unroll
        for (int r = 0; r < kRows; r++) {
            float x[8];
            const float *src = q + (size_t)(r0 + min((uint32_t)r, nr - 1)) * 4096 + (g * 8 + h) * 256 + d0;
#pragma unroll
            for (int e = 0; e < 8; e++) x[e] = src[e];   // (the query binding needs only 4-byte alignment)
            float amax = 0.0f;
#pragma unroll
            for (int e = 0; e < 8; e++) amax = fmaxf(amax, fabsf(x[e]));
#pragma unroll
            for (int o = 16; o > 0; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o, 64));   // the head's 32 lanes
            const float inv = amax > 0.0f ? 127.0f / amax : 0.0f;
            if ((tid & 31) == 0) qscale[r][h] = amax * (1.0f / 127.0f);
            uint32_t w1[2] = {0, 0}, w2[2] = {0, 0}, w3[2] = {0, 0};
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const float z = x[e] * inv, q1 = rintf(z), r1 = z - q1;
                const float q2 = rintf(r1 * 254.0f);
                const float r2 = fmaf(r1, 254.0f, -q2);
                const float q3 = rintf(r2 * 254.0f);
                w1[e >> 2] |= code(q1) << (8 * (e & 3));
                w2[e >> 2] |= code(q2) << (8 * (e & 3));
                w3[e >> 2] |= code(q3) << (8 * (e & 3));
            }
            // dimension d0 + e is byte (d0 % 16) + e of lane 16 ((d0 % 64) / 16) + column of step d0 / 64
            const int step = d0 >> 6, at = 16 * ((d0 & 63) >> 4), half = (d0 & 15) >> 3;
            unsigned char *base = reinterpret_cast<unsigned char *>(&qop[r][0][step][0]);
            *reinterpret_cast<uint2 *>(base + (at + h) * 16 + 8 * half) = make_uint2(w1[0], w1[1]);
            *reinterpret_cast<uint2 *>(base + (at + h + 8) * 16 + 8 * half) = make_uint2(w2[0], w2[1]);
            unsigned char *base3 = reinterpret_cast<unsigned char *>(&qop[r][1][step][0]);
            *reinterpret_cast<uint2 *>(base3 + (at + h) * 16 + 8 * half) = make_uint2(w3[0], w3[1]);
            *reinterpret_cast<uint2 *>(base3 + (at + h + 8) * 16 + 8 * half) = make_uint2(w3[0], w3[1]);
        }
    }
    __syncthreads();
    const bool lo_col = n >= 8;
    // Two 16-token tiles at a time: after the hi/lo exchange lanes n < 8 finish the first and lanes
    // n >= 8 the second, so that one store instruction writes 128 contiguous bytes of each head's row
    // with every lane active. The work-group's `span` tokens (256 or 512) are split over the waves.
    const uint32_t per_wave = span / 4;
#pragma unroll 1
    for (uint32_t tp = 0; tp < per_wave / 32; tp++) {
        const uint32_t ta = kt * span + per_wave * wave + 32 * tp;
        if (ta >= K) break;   // wave-uniform
        v4i kop[2][4];
        float kss[2][4];
#pragma unroll
        for (int u = 0; u < 2; u++) {
            const uint32_t tk = min(ta + 16 * u + n, length - 1);   // the lane's K row (an existing one)
#pragma unroll
            for (int jj = 0; jj < 4; jj++)
                kop[u][jj] = *reinterpret_cast<const v4i *>(k + ((size_t)tk * 2 + g) * 256 + 64 * jj + 16 * qq);
#pragma unroll
            for (int i = 0; i < 4; i++) kss[u][i] = ks[(size_t)min(ta + 16 * u + 4 * qq + i, length - 1) * 2 + g];
        }
        const uint32_t tb = ta + (lo_col ? 16 : 0);   // the tile this lane finishes
#pragma unroll
        for (int r = 0; r < kRows; r++) {
            if ((uint32_t)r >= nr) break;   // uniform
            v4i acc[2] = {{0, 0, 0, 0}, {0, 0, 0, 0}}, acc3[2] = {{0, 0, 0, 0}, {0, 0, 0, 0}};
#pragma unroll
            for (int u = 0; u < 2; u++)
#pragma unroll
                for (int jj = 0; jj < 4; jj++) {
                    acc[u] = __builtin_amdgcn_mfma_i32_16x16x64_i8(kop[u][jj], qop[r][0][jj][lane], acc[u], 0, 0, 0);
                    acc3[u] = __builtin_amdgcn_mfma_i32_16x16x64_i8(kop[u][jj], qop[r][1][jj][lane], acc3[u], 0, 0, 0);
                }
            // column n holds head n % 8's part q1 (n < 8) or q2 (n >= 8), both columns its q3; token
            // tb + 4qq + i of this lane's tile
            const float qsc = qscale[r][n & 7];
            const uint32_t last = pos + r0 + r;   // the row's last visible key
            float *dst = scores + ((size_t)(r0 + r) * 16 + g * 8 + (n & 7)) * K;
            float out[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int ma = acc[0][i], oa = __shfl_xor(ma, 8, 64);
                const int mb = acc[1][i], ob = __shfl_xor(mb, 8, 64);
                const float hi = (float)(lo_col ? ob : ma), lo = (float)(lo_col ? mb : oa);
                const int c3 = lo_col ? acc3[1][i] : acc3[0][i];
                const float full = fmaf((float)c3, 1.0f / 64516.0f, fmaf(lo, 1.0f / 254.0f, hi)) * qsc;
                const uint32_t t = tb + 4 * qq + i;
                out[i] = t <= last ? full * (lo_col ? kss[1][i] : kss[0][i]) * (1.0f / 16.0f) : -INFINITY;
            }
            // the lane's four consecutive tokens as one 16-byte store where the row allows it
            const uint32_t t4 = tb + 4 * qq;
            if (t4 + 3 < K && (reinterpret_cast<uintptr_t>(dst + t4) & 15) == 0) {
                *reinterpret_cast<float4 *>(dst + t4) = make_float4(out[0], out[1], out[2], out[3]);
            } else {
#pragma unroll
                for (int i = 0; i < 4; i++)
                    if (t4 + i < K) dst[t4 + i] = out[i];
            }
        }
    }
}

__device__ inline float block_reduce_256(float v, float *partial, bool is_max) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        float other = __shfl_xor(v, o, 64);
        v = is_max ? fmaxf(v, other) : v + other;
    }
    __syncthreads();
    if ((threadIdx.x & 63) == 0) partial[threadIdx.x >> 6] = v;
    __syncthreads();
    float r = partial[0];
    for (int i = 1; i < 4; i++) r = is_max ? fmaxf(r, partial[i]) : r + partial[i];
    return r;
}

// In-place softmax over i <= pos of each row of stride K (kernels.metal:163-166), in two passes
// over chunks of kSoftmaxChunk elements (absolute boundaries, so that a row's result does not
// depend on how many rows the dispatch holds): the chunk's maximum and its sum of exp(x - max),
// then, per chunk, the row's maximum M and sum L merged from those in chunk order and
// x = exp(x - M) / L. Elements past pos are left as they are.
constexpr int kSoftmaxChunk = 8192;
constexpr int kSoftmaxPer = kSoftmaxChunk / 256;

__global__ __launch_bounds__(256) void softmax_stats_kernel(const float *__restrict__ x, float2 *__restrict__ stats,
                                                            uint32_t K, uint32_t pos, uint32_t chunks) {
    __shared__ float partial[4];
    const uint32_t c = blockIdx.x, r = blockIdx.y;
    const float *row = x + (size_t)r * K;
    const uint32_t lo = c * kSoftmaxChunk, hi = min(pos + 1, lo + kSoftmaxChunk);
    // every chunk holds at least one element at or below pos: loads of a clamped index, then the
    // elements past the row's end are masked (no branch per load)
    float e[kSoftmaxPer];
#pragma unroll
    for (int j = 0; j < kSoftmaxPer; j++) e[j] = row[min(lo + threadIdx.x + 256 * j, hi - 1)];
#pragma unroll
    for (int j = 0; j < kSoftmaxPer; j++)
        if (lo + threadIdx.x + 256 * j >= hi) e[j] = -INFINITY;
    float top = -INFINITY;
#pragma unroll
    for (int j = 0; j < kSoftmaxPer; j++) top = fmaxf(top, e[j]);
    top = block_reduce_256(top, partial, true);
    float sum = 0.0f;
    if (top != -INFINITY)
#pragma unroll
        for (int j = 0; j < kSoftmaxPer; j++) sum += expf(e[j] - top);
    sum = block_reduce_256(sum, partial, false);
    if (threadIdx.x == 0) stats[(size_t)r * chunks + c] = make_float2(top, sum);
}

__global__ __launch_bounds__(256) void softmax_apply_kernel(float *__restrict__ x, const float2 *__restrict__ stats,
                                                            uint32_t K, uint32_t pos, uint32_t chunks) {
    const uint32_t c = blockIdx.x, r = blockIdx.y;
    // the chunk's loads go out first; the row's statistics (the same for the whole work-group)
    // are merged while they are in flight
    float *row = x + (size_t)r * K;
    const uint32_t lo = c * kSoftmaxChunk, hi = min(pos + 1, lo + kSoftmaxChunk);
    float e[kSoftmaxPer];
#pragma unroll
    for (int j = 0; j < kSoftmaxPer; j++) e[j] = row[min(lo + threadIdx.x + 256 * j, hi - 1)];
    const float2 *st = stats + (size_t)r * chunks;
    float top = -INFINITY;
    for (uint32_t k = 0; k < chunks; k++) top = fmaxf(top, st[k].x);
    float sum = 0.0f;
    for (uint32_t k = 0; k < chunks; k++)
        if (st[k].x != -INFINITY) sum += st[k].y * expf(st[k].x - top);
    if (hi == lo + kSoftmaxChunk) {   // a whole chunk: no mask per store
#pragma unroll
        for (int j = 0; j < kSoftmaxPer; j++) row[lo + threadIdx.x + 256 * j] = expf(e[j] - top) / sum;
    } else {
#pragma unroll
        for (int j = 0; j < kSoftmaxPer; j++) {
            const uint32_t i = lo + threadIdx.x + 256 * j;
            if (i < hi) row[i] = expf(e[j] - top) / sum;
        }
    }
}

// y[(row*16+h)*256+d] = sum_{t <= pos+row} scores*vs*vcode * sigmoid(gate) (kernels.metal:153-156),
// split over absolute kValuesSplit-token ranges (a row's sum does not depend on the dispatch's
// row count); values_combine_kernel adds the splits in order and applies the gate.
constexpr int kValuesSplit = 512;

// Work-group (split, KV group, kRows rows): O^T[d][c] += V^T[d][t] B[t][c] on
// v_mfma_f32_16x16x16_f16 with the codes exact in FP16 and, per row, B = p * vs * 2^15 / vs_r in
// the 16 columns 8 heads x {FP16 hi, FP16 lo} (vs_r the row's largest V scale over its tokens of
// the split, so that B <= 2^15; hi + lo keeps about 22 bits), the result times vs_r / 2^15. The
// factor 2^15 keeps the probabilities of a long, flat row (p ~ 1 / K) out of FP16's subnormals
// (below 2^-14), where hi and lo would keep only a few bits. Eight waves, wave w taking
// dimensions 32w .. 32w + 31 (96 registers: two work-groups per CU; four waves with 64 dimensions
// each held 168, three per CU, 21.5 against 18.9 us at 4 rows over 30000 keys); a 64-token block
// is four k-steps, lane (n, qq) of step s holding tokens 16qq + 4s .. + 3 of the block for both
// operands (one 16-byte code load per dimension tile covers its four steps), and the next block's
// loads are issued before the current block is staged. Every quantity of a row depends on that
// row's range only, whatever kRows is.
constexpr int kVmBlock = 64;
constexpr float kValuesScale = 32768.0f;   // 2^15: B's factor

template <int kRows>
__global__ __launch_bounds__(512) void values_partial_kernel(const float *__restrict__ scores,
                                                             const int8_t *__restrict__ v, const float *__restrict__ vs,
                                                             float *__restrict__ partial, uint32_t rows, uint32_t K,
                                                             uint32_t pos, uint32_t splits, uint32_t zs) {
    typedef _Float16 half4 __attribute__((ext_vector_type(4)));
    constexpr int kWaves = 8;                           // wave w: dimensions 32w .. 32w + 31
    // B operands [row][k-step][slot]: lane L's operand in slot L ^ ((L / 16) % 4 * 2), each k-step row
    // padded by one slot. A staging store writes one (row, head)'s 64 tokens, which fall in 16
    // slots (4 k-steps x 4 token blocks); without the padding and the XOR the four k-steps (512 bytes
    // apart) and token blocks 0 and 2 share their banks, 8 to 16 lanes per bank; with them the 16
    // slots cover 32 banks. The operand reads (64 slots of one k-step row) stay conflict-free.
    __shared__ uint2 bs[kRows][4][65];
    auto bslot = [](int L) __attribute__((always_inline)) { return L ^ ((L >> 3) & 6); };
    __shared__ float vred[kWaves][kRows];
    // the row blocks of one (split, group) pair 8 blocks apart: one XCD reads the pair's V once
    const uint32_t xcd = blockIdx.x % 8, jb = blockIdx.x / 8, pair = (jb / zs) * 8 + xcd;
    if (pair >= 2 * splits) return;   // padding of the grid to whole rounds of 8
    const uint32_t split = pair / 2, g = pair % 2, r0 = (jb % zs) * kRows;
    const uint32_t nr = min((uint32_t)kRows, rows - r0);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, n = lane & 15, qq = lane >> 4;
    const uint32_t t0 = split * kValuesSplit;
    const uint32_t t1 = min(pos + r0 + nr, t0 + kValuesSplit);   // the work-group's last row's end
    // each row's largest V scale over its tokens of the split
    float vr[kRows];
    {
        float vm[kRows];
#pragma unroll
        for (int r = 0; r < kRows; r++) vm[r] = 0.0f;
        if (t0 < t1)
#pragma unroll
            for (int k = 0; k < kValuesSplit / 512; k++) {
                const uint32_t t = t0 + tid + 512 * k;
                const float x = vs[(size_t)min(t, t1 - 1) * 2 + g];
#pragma unroll
                for (int r = 0; r < kRows; r++)
                    if (t < pos + r0 + r + 1) vm[r] = fmaxf(vm[r], x);
            }
#pragma unroll
        for (int r = 0; r < kRows; r++) {
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) vm[r] = fmaxf(vm[r], __shfl_xor(vm[r], o, 64));
            if (lane == 0) vred[wave][r] = vm[r];
        }
        __syncthreads();
#pragma unroll
        for (int r = 0; r < kRows; r++) {
            vr[r] = vred[0][r];
#pragma unroll
            for (int w = 1; w < kWaves; w++) vr[r] = fmaxf(vr[r], vred[w][r]);
        }
    }
    floatx4 acc[2][kRows];
#pragma unroll
    for (int dt = 0; dt < 2; dt++)
#pragma unroll
        for (int r = 0; r < kRows; r++) acc[dt][r] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    // staging: thread T takes token T % 64 of the block for row i, head T / 64 (the wave: uniform) of
    // every row i, so that a wave's score loads read 64 consecutive tokens of one (row, head). The
    // loads are unconditional (row and token clamped into the rows and keys that exist) and the
    // causal mask a select at staging time (a select at the load would wait for it there), so no
    // load sits under a per-lane branch.
    const int tok = tid & 63, sh = __builtin_amdgcn_readfirstlane(tid >> 6);
    struct Loads {
        float sc[kRows], sv;
        uint4 w4[2];   // the wave's two dimension tiles: dimension 32 wave + 16 dt + n, tokens 16 qq .. + 15
    };
    auto load = [&](Loads &L, uint32_t tb) __attribute__((always_inline)) {
        const uint32_t t = tb + tok, tc = min(t, t1 - 1);
        L.sv = vs[(size_t)tc * 2 + g];
#pragma unroll
        for (int i = 0; i < kRows; i++) {
            const uint32_t rc = min((uint32_t)i, nr - 1);
            L.sc[i] = scores[((size_t)(r0 + rc) * 16 + g * 8 + sh) * K + tc];
        }
#pragma unroll
        for (int dt = 0; dt < 2; dt++)
            L.w4[dt] = *reinterpret_cast<const uint4 *>(v + value_index((uint64_t)tb * 2 + g, 32 * wave + 16 * dt + n) + 16 * qq);
    };
    Loads cur, nxt;
    if (t0 < t1) load(cur, t0);
    for (uint32_t tb = t0; tb < t1; tb += kVmBlock) {
        const bool more = tb + kVmBlock < t1;   // work-group-uniform
        if (more) load(nxt, tb + kVmBlock);
        __syncthreads();   // the previous block's B reads are done
        {
            // token tok of the block is k = 4 (tok / 16) + tok % 4 of step (tok % 16) / 4: half tok % 4
            // of lane 16 (tok / 16) + column
            const int s = (tok & 15) >> 2, j = tok & 3, lrow = 16 * (tok >> 4);
#pragma unroll
            for (int i = 0; i < kRows; i++) {
                if ((uint32_t)i < nr) {   // uniform
                    const float inv = vr[i] > 0.0f ? kValuesScale / vr[i] : 0.0f;
                    const float p = tb + tok < pos + r0 + i + 1 ? cur.sc[i] : 0.0f;   // the causal mask
                    const float x = p * cur.sv * inv;
                    const _Float16 hi = (_Float16)x, lo = (_Float16)(x - (float)hi);
                    reinterpret_cast<_Float16 *>(&bs[i][s][bslot(lrow + sh)])[j] = hi;
                    reinterpret_cast<_Float16 *>(&bs[i][s][bslot(lrow + sh + 8)])[j] = lo;
                }
            }
        }
        __syncthreads();
#pragma unroll
        for (int s = 0; s < 4; s++) {
            half4 a[2];
#pragma unroll
            for (int dt = 0; dt < 2; dt++) {
                const uint4 &w = cur.w4[dt];
                const uint32_t word = s == 0 ? w.x : s == 1 ? w.y : s == 2 ? w.z : w.w;
                uint32_t h0, h1;
                i8x4_to_f16(word, h0, h1);
                a[dt] = __builtin_bit_cast(half4, make_uint2(h0, h1));
            }
#pragma unroll
            for (int r = 0; r < kRows; r++) {
                if ((uint32_t)r >= nr) break;   // uniform
                const half4 b = __builtin_bit_cast(half4, bs[r][s][bslot(lane)]);
#pragma unroll
                for (int dt = 0; dt < 2; dt++) acc[dt][r] = __builtin_amdgcn_mfma_f32_16x16x16f16(a[dt], b, acc[dt][r], 0, 0, 0);
            }
        }
        if (more) cur = nxt;
    }
    // the lo column n + 8 joins the hi column n (head n); lanes n < 8 write dimensions 32 wave + 16 dt + 4 qq + e
#pragma unroll
    for (int r = 0; r < kRows; r++) {
        if ((uint32_t)r >= nr) break;
        float *out = partial + (((size_t)(r0 + r) * 2 + g) * splits + split) * 2048;
        const float f = vr[r] * (1.0f / kValuesScale);   // exact: a power of two
#pragma unroll
        for (int dt = 0; dt < 2; dt++) {
            float4 o4;
            o4.x = (acc[dt][r][0] + __shfl_xor(acc[dt][r][0], 8, 64)) * f;
            o4.y = (acc[dt][r][1] + __shfl_xor(acc[dt][r][1], 8, 64)) * f;
            o4.z = (acc[dt][r][2] + __shfl_xor(acc[dt][r][2], 8, 64)) * f;
            o4.w = (acc[dt][r][3] + __shfl_xor(acc[dt][r][3], 8, 64)) * f;
            if (n < 8) *reinterpret_cast<float4 *>(out + n * 256 + 32 * wave + 16 * dt + 4 * qq) = o4;
        }
    }
}

__global__ __launch_bounds__(64) void values_combine_kernel(const float *__restrict__ partial,
                                                             const float *__restrict__ gate, float *__restrict__ y,
                                                             uint32_t splits) {
    const uint32_t h = blockIdx.x / 4, row = blockIdx.y, g = h / 8, d = 64 * (blockIdx.x % 4) + threadIdx.x;
    const float *src = partial + ((size_t)row * 2 + g) * splits * 2048 + (h % 8) * 256 + d;
    float sum = 0.0f;
    for (uint32_t s = 0; s < splits; s += 32) {   // 32 loads in flight, added in split order
        float x[32];
#pragma unroll
        for (int u = 0; u < 32; u++) x[u] = src[(size_t)min(s + u, splits - 1) * 2048];
#pragma unroll
        for (int u = 0; u < 32; u++)
            if (s + u < splits) sum += x[u];
    }
    const size_t i = ((size_t)row * 16 + h) * 256 + d;
    y[i] = sum * (1.0f / (1.0f + expf(-gate[i])));
}

// ---------------------------------------------------------------- fused split-K decode

constexpr int kChunk = 128;                      // tokens per LDS chunk (one 128-byte line per V page row)
constexpr int kDecodeWaves = 8;
constexpr int kMaxSplitTokens = 2048;            // tokens per work-group at most (LDS scales)
constexpr int kPartialFloats = 8 * 256 + 16;    // O[8][256], m[8], l[8] per (row, group, split)
constexpr int kMaxDecodeSplits = 1024;
constexpr float kLog2e = 1.4426950408889634f;

struct DecodeParams {
    const float *q;              // FP32 [rows][16][256] (or qh below)
    const int8_t *k;
    const int8_t *v;
    const float *ks;
    const float *vs;
    const float *gate;
    float *y;
    float *partial;
    uint32_t rows, pos, splits;
    uint32_t split_chunks;   // 128-token chunks per split
    // attention_decode_append_int8 (one row): q is the unrotated query; the kernel rotates it
    // (writing it to `rotated`), quantizes the new token's K (rotated) and V into the cache at
    // `pos` (k_out, v_out, ks_out, vs_out alias k, v, ks, vs) and attends over it
    uint32_t append;
    RopeFreq freq;
    const float *knew, *vnew;    // FP32 [2][256] each
    float *rotated;              // FP32 [16][256]
    int8_t *k_out, *v_out;
    float *ks_out, *vs_out;
    const _Float16 *qh;          // prefill chunks routed here: the grouped FP16 query [2][rows][8][256]
};

// sigmoid(x) = 1 / (1 + 2^(-x log2(e))) with the hardware exponential and reciprocal (about an ulp
// each), as the prefill kernels compute it
// x of lane l ^ 16 (v_permlane16_swap) and of lane l ^ 32 (v_permlane32_swap) added or maxed in:
// with both operands holding x, every lane ends with its own value in one register and its
// partner's in the other; the no-ops cover the cross-lane move's wait states. Registers, not an
// LDS round trip as a shuffle takes.
__device__ inline float xl_sum16(float x) {
    float a = x, b = x;
    asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
    return a + b;
}
__device__ inline float xl_sum32(float x) {
    float a = x, b = x;
    asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
    return a + b;
}
__device__ inline float xl_max16(float x) {
    float a = x, b = x;
    asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
    return fmaxf(a, b);
}
__device__ inline float xl_max32(float x) {
    float a = x, b = x;
    asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
    return fmaxf(a, b);
}
// x of lane l ^ 8 (the other half of its 16-lane row) by a DPP rotation of the row by 8
__device__ inline float xl_swap8(float x) {
    float y;
    asm volatile("s_nop 1\n\tv_mov_b32_dpp %0, %1 row_ror:8 row_mask:0xf bank_mask:0xf" : "=v"(y) : "v"(x));
    return y;
}

__device__ inline float sigmoidf(float x) {
    return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-x * 1.4426950408889634f));
}

// x + x of lane l ^ 8 (the same position in the other half of its 16-lane row) for
// the eight values of two accumulators: one DPP add each, as inline assembly (the DPP
// move builtin was mis-scheduled here, and a cross-lane shuffle costs an LDS round
// trip per value). The sources are MFMA results whose wait states the caller has
// covered and no add reads another's result, so only the block's ends need wait
// states (a register copy the compiler places just before the block).
__device__ inline void add_row_partner8(floatx4 &a, floatx4 &b) {
    float r0, r1, r2, r3, r4, r5, r6, r7;
    asm volatile(
        "s_nop 1\n\t"
        "v_add_f32_dpp %0, %8, %8 row_ror:8 row_mask:0xf bank_mask:0xf\n\t"
        "v_add_f32_dpp %1, %9, %9 row_ror:8 row_mask:0xf bank_mask:0xf\n\t"
        "v_add_f32_dpp %2, %10, %10 row_ror:8 row_mask:0xf bank_mask:0xf\n\t"
        "v_add_f32_dpp %3, %11, %11 row_ror:8 row_mask:0xf bank_mask:0xf\n\t"
        "v_add_f32_dpp %4, %12, %12 row_ror:8 row_mask:0xf bank_mask:0xf\n\t"
        "v_add_f32_dpp %5, %13, %13 row_ror:8 row_mask:0xf bank_mask:0xf\n\t"
        "v_add_f32_dpp %6, %14, %14 row_ror:8 row_mask:0xf bank_mask:0xf\n\t"
        "v_add_f32_dpp %7, %15, %15 row_ror:8 row_mask:0xf bank_mask:0xf\n\t"
        "s_nop 1"
        : "=&v"(r0), "=&v"(r1), "=&v"(r2), "=&v"(r3), "=&v"(r4), "=&v"(r5), "=&v"(r6), "=&v"(r7)
        : "v"(a[0]), "v"(a[1]), "v"(a[2]), "v"(a[3]), "v"(b[0]), "v"(b[1]), "v"(b[2]), "v"(b[3]));
    a = floatx4{r0, r1, r2, r3};
    b = floatx4{r4, r5, r6, r7};
}

// One chunk of one KV group in flight, K and V in separate register sets (K is staged
// one chunk ahead of V): thread t holds K rows t / 16 + 32 i (16 bytes at 16 (t % 16))
// and V page-row segments t / 8 + 64 i (16 bytes at 16 (t % 8)), i < 4: every load
// instruction reads whole 256-byte K rows or whole 128-byte V lines, the pattern that
// streams at full HBM rate (loads shaped like the MFMA operands, 16 rows per
// instruction, reach about two thirds of it).
struct KRegs {
    uint4 k0, k1, k2, k3;   // named, not an array: kept in registers
};
struct VRegs {
    uint4 v0, v1, v2, v3;
};

// The LDS image of a chunk. K: 128 token rows of 256 bytes, 16-byte piece c of
// token t at position c ^ (t % 16). V^T: 256 dimension rows of 128 bytes (the
// chunk's tokens), piece c (tokens 16c..16c+15) of row d at position c ^ ((d / 2) % 8).
// Both make the operand reads and the chunk writes free of bank conflicts.
struct ChunkLds {
    uint4 k[kChunk][16];
    uint4 v[256][8];
};

// The chunk loads are non-temporal (`nt`): each cache byte is read once per step, so it need not
// displace anything in L2 (29.5 instead of 30.6-31.1 us per layer step at 131073).
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

__device__ __attribute__((always_inline)) inline uint4 load_k_piece(const DecodeParams &p, uint32_t g, uint32_t c0,
                                                                    uint32_t length, int tid, int i) {
    const uint32_t t = min(c0 + (uint32_t)(tid >> 4) + 32 * i, length - 1);
    return __builtin_bit_cast(
        uint4, __builtin_nontemporal_load(reinterpret_cast<const u32x4_t *>(p.k + ((size_t)t * 2 + g) * 256 + 16 * (tid & 15))));
}

// 16 bytes as a value (a struct copy straight from global memory would keep the
// register set in a stack object)
__device__ __attribute__((always_inline)) inline uint4 load_piece(const int8_t *at) {
    return __builtin_bit_cast(uint4, __builtin_nontemporal_load(reinterpret_cast<const u32x4_t *>(at)));
}

// K or V of chunk idx of the split starting at token `begin`. Past the last chunk
// (only the prologue's loads of a split shorter than three chunks) the loads stay, a
// fixed count that keeps the counter waits exact, but every lane reads the same 16
// bytes of the first one: a cache line instead of a 32 KB re-read.
__device__ __attribute__((always_inline)) inline void load_k(KRegs &r, const DecodeParams &p, uint32_t g,
                                                             uint32_t begin, uint32_t idx, uint32_t nchunks,
                                                             uint32_t length, int tid) {
    const bool real = idx < nchunks;
    const uint32_t c0 = real ? begin + idx * kChunk : begin;
    const int lt = real ? tid : 0;
    r.k0 = load_k_piece(p, g, c0, length, lt, 0);
    r.k1 = load_k_piece(p, g, c0, length, lt, real ? 1 : 0);
    r.k2 = load_k_piece(p, g, c0, length, lt, real ? 2 : 0);
    r.k3 = load_k_piece(p, g, c0, length, lt, real ? 3 : 0);
}

__device__ __attribute__((always_inline)) inline void load_v(VRegs &r, const DecodeParams &p, uint32_t g,
                                                             uint32_t begin, uint32_t idx, uint32_t nchunks,
                                                             int tid) {
    const bool real = idx < nchunks;
    const uint32_t c0 = real ? begin + idx * kChunk : begin;
    const int lt = real ? tid : 0;
    // c0 is a multiple of 128 inside the cache's whole pages
    const int8_t *vrow = p.v + value_index((uint64_t)c0 * 2 + g, 0) + (size_t)(lt >> 3) * 256 + 16 * (lt & 7);
    const size_t step = real ? 64 * 256 : 0;
    r.v0 = load_piece(vrow);
    r.v1 = load_piece(vrow + step);
    r.v2 = load_piece(vrow + 2 * step);
    r.v3 = load_piece(vrow + 3 * step);
}

__device__ __attribute__((always_inline)) inline void store_k(ChunkLds &b, const KRegs &r, int tid) {
    const int t = tid >> 4, c = tid & 15;   // K rows t + 32i (t + 32i has the same t % 16)
    const int kp = c ^ (t & 15);
    b.k[t][kp] = r.k0;
    b.k[t + 32][kp] = r.k1;
    b.k[t + 64][kp] = r.k2;
    b.k[t + 96][kp] = r.k3;
}

__device__ __attribute__((always_inline)) inline void store_v(ChunkLds &b, const VRegs &r, int tid) {
    const int d = tid >> 3, e = tid & 7;    // V rows d + 64i (same (d / 2) % 8)
    const int vp = e ^ ((d >> 1) & 7);
    b.v[d][vp] = r.v0;
    b.v[d + 64][vp] = r.v1;
    b.v[d + 128][vp] = r.v2;
    b.v[d + 192][vp] = r.v3;
}

// The appended token's bytes in a chunk's registers, just before they are staged: K row `tn` of
// the chunk (held by the 16 threads with tid / 16 == tn % 32, piece tid % 16, in register
// tn / 32) and byte tn % 16 of the 16-token segment tn / 16 of every V page row (threads with
// tid % 8 == tn / 16, rows tid / 8 + 64 i). Whatever the loads returned for that position is
// replaced by the freshly quantized codes.
// (selections are made on 32-bit words with masks: a select between whole uint4 values became a
// select between their addresses and sent the register sets to scratch)
__device__ __attribute__((always_inline)) inline void take_if(uint4 &w, uint32_t keep, const uint4 &f) {
    w.x = (w.x & keep) | (f.x & ~keep);
    w.y = (w.y & keep) | (f.y & ~keep);
    w.z = (w.z & keep) | (f.z & ~keep);
    w.w = (w.w & keep) | (f.w & ~keep);
}

__device__ __attribute__((always_inline)) inline void patch_k(KRegs &r, int tid, int tn, const uint4 *fresh) {
    if ((tid >> 4) != (tn & 31)) return;
    const uint4 f = fresh[tid & 15];
    const int i = tn >> 5;
    take_if(r.k0, i == 0 ? 0u : ~0u, f);
    take_if(r.k1, i == 1 ? 0u : ~0u, f);
    take_if(r.k2, i == 2 ? 0u : ~0u, f);
    take_if(r.k3, i == 3 ? 0u : ~0u, f);
}

__device__ __attribute__((always_inline)) inline uint4 patch_byte(uint4 w, int byte, uint32_t code) {
    const uint32_t sh = 8 * (byte & 3), value = (code & 0xffu) << sh;
    const int word = byte >> 2;
    const uint32_t m0 = word == 0 ? 0xffu << sh : 0u, m1 = word == 1 ? 0xffu << sh : 0u;
    const uint32_t m2 = word == 2 ? 0xffu << sh : 0u, m3 = word == 3 ? 0xffu << sh : 0u;
    w.x = (w.x & ~m0) | (value & m0);
    w.y = (w.y & ~m1) | (value & m1);
    w.z = (w.z & ~m2) | (value & m2);
    w.w = (w.w & ~m3) | (value & m3);
    return w;
}

__device__ __attribute__((always_inline)) inline void patch_v(VRegs &r, int tid, int tn, const uint8_t *fresh) {
    if ((tid & 7) != (tn >> 4)) return;
    const int d = tid >> 3, byte = tn & 15;
    r.v0 = patch_byte(r.v0, byte, fresh[d]);
    r.v1 = patch_byte(r.v1, byte, fresh[d + 64]);
    r.v2 = patch_byte(r.v2, byte, fresh[d + 128]);
    r.v3 = patch_byte(r.v3, byte, fresh[d + 192]);
}

// Grid: (splits, 2 KV groups, rows), one 8-wave work-group per CU; a split is
// split_chunks chunks of 128 tokens, chosen on the host so that the grid fits the
// CUs in one round. The work-group streams its chunks through double-buffered LDS
// with two chunks in flight in registers. Per chunk wave w scores tokens 16w..16w+15,
// S^T[t][n] = K[t] . Qx[n] (16x16x64 INT8 MFMA on the raw K codes, n = 8 heads x
// {q1, q2}, and a second product for q3), and turns them into probabilities in base 2 against a running reference
// shared by the work-group; the waves exchange those P operands through LDS and wave w
// accumulates O^T[d][n] += V^T[d][t] . Px[t][n] for dimensions 32w..32w+31 over all 128
// tokens (16x16x32 FP16 MFMA), so no wave merge of O remains at the end. Px = p * vs /
// vs_ref split into FP16 hi + lo; vs_ref, the split's largest V scale, keeps Px below
// 256 and multiplies the result once. Lane l holds MFMA column n = l % 16 and
// token/k group qq = l / 16.
template <bool kHalfQ>
__global__ __launch_bounds__(512, 1) void decode_int8_kernel(DecodeParams p) {
    typedef int v4i __attribute__((ext_vector_type(4)));
    typedef _Float16 half4 __attribute__((ext_vector_type(4)));
    // the chunk buffers
    __shared__ __attribute__((aligned(16))) unsigned char arena[2 * sizeof(ChunkLds)];
    ChunkLds *bufs = reinterpret_cast<ChunkLds *>(arena);
    __shared__ float chunk_top[2][kDecodeWaves][16], wave_l[kDecodeWaves][16];
    __shared__ uint2 pshare[2][kDecodeWaves][64];   // each wave's P operands, by chunk parity
    __shared__ float kscale[kMaxSplitTokens], vscale[kMaxSplitTokens];
    __shared__ float red[kDecodeWaves], qmax[4][8];
    // append mode: rotated dims 0..63 of the group's 8 query heads, and the new token's codes
    // (K row, V column) and scales
    __shared__ __attribute__((aligned(16))) float qrot0[8][64];
    __shared__ __attribute__((aligned(16))) uint8_t fresh_k[256], fresh_v[256];
    __shared__ float fresh_scale[2];
    // INT8 query operands [set][MFMA c][lane] (set 0: q1 | q2 columns, set 1: q3), built once
    // and read into registers before the chunk loop. They sit in the V half of chunk buffer
    // 1, which is first written in phase 1, after the barrier that ends phase 0: by then every
    // wave has read its operands.
    v4i(*qlds)[4][64] = reinterpret_cast<v4i(*)[4][64]>(&bufs[1].v[0][0]);
    static_assert(2 * 4 * 64 * sizeof(v4i) <= sizeof(ChunkLds::v), "query operands exceed the V half of a buffer");
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n = lane & 15, qq = lane >> 4, head = n & 7;
    const bool lo_col = n >= 8;
    const uint32_t split = blockIdx.x, g = blockIdx.y, row = blockIdx.z;
    const uint32_t length = p.pos + row + 1;
    const uint32_t split_tokens = p.split_chunks * kChunk;
    const uint32_t begin = split * split_tokens;
    const uint32_t end = min(length, begin + split_tokens);
    const uint32_t nchunks = end > begin ? (end - begin + kChunk - 1) / kChunk : 0;
    // append mode: the split holding the new token (position pos) stages fresh codes for it
    const bool owner = p.append && begin <= p.pos && p.pos < end;
    const int e_new = owner ? (int)(p.pos - begin) : -1;          // split-local index
    const int jn = owner ? e_new / kChunk : -1, tn = owner ? e_new % kChunk : 0;

    // ---- the small loads first (scales of the split, this wave's query chunk), then
    // the first two chunks: waits on the memory counter are in order, so the set-up
    // below never waits for the chunks
    // (a fixed count of loads, no branches: the counter waits below stay exact;
    // indices past the split repeat its last token, a cache hit)
    uint32_t last = (end > begin ? end : length) - 1;
    if (p.append && last == p.pos && p.pos > 0) last = p.pos - 1;   // its stored scales are stale
    float ksv[kMaxSplitTokens / 512], vsv[kMaxSplitTokens / 512];
#pragma unroll
    for (int it = 0; it < kMaxSplitTokens / 512; it++) {
        const size_t at = (size_t)min(begin + tid + 512 * it, last) * 2 + g;
        ksv[it] = p.ks[at];
        vsv[it] = p.vs[at];
    }
    // query chunk c = wave % 4: lane (n, qq) takes dims 64c + 16qq + [0, 16) of head
    // n % 8 (waves 4-7 load the same chunks and only waves 0-3 publish them)
    const int chunk = wave & 3;
    float4 x[4];
    if constexpr (kHalfQ) {
        // the prefill path's grouped FP16 query, [(g rows + row) 8 + head][256]: exact in FP32
        const _Float16 *qs = p.qh + (((size_t)g * p.rows + row) * 8 + head) * 256 + 64 * chunk + 16 * qq;
        const half8 a = *reinterpret_cast<const half8 *>(qs), b = *reinterpret_cast<const half8 *>(qs + 8);
        x[0] = make_float4((float)a[0], (float)a[1], (float)a[2], (float)a[3]);
        x[1] = make_float4((float)a[4], (float)a[5], (float)a[6], (float)a[7]);
        x[2] = make_float4((float)b[0], (float)b[1], (float)b[2], (float)b[3]);
        x[3] = make_float4((float)b[4], (float)b[5], (float)b[6], (float)b[7]);
    } else {
        const float *qs = p.q + ((size_t)row * 16 + g * 8 + head) * 256 + 64 * chunk + 16 * qq;
#pragma unroll
        for (int f = 0; f < 4; f++) x[f] = *reinterpret_cast<const float4 *>(qs + 4 * f);
    }
    // append mode: head `wave` of the group in rope4's layout (dims 4 lane .. +3) and the new
    // token's K and V of the group. Loaded in every mode and every wave (from the query itself
    // when there is no new token): a fixed count of loads keeps the counter waits exact.
    // (the FP16 query path has no FP32 query and no new token: its first 2 KB, in range for any
    // row count, stand in for these unused loads)
    const float *qf = kHalfQ ? reinterpret_cast<const float *>(p.qh) : p.q;
    const float *knew = p.append ? p.knew : qf, *vnew = p.append ? p.vnew : qf;
    const float4 rq = *reinterpret_cast<const float4 *>(
        kHalfQ ? qf + 4 * lane : p.q + ((size_t)row * 16 + g * 8 + wave) * 256 + 4 * lane);
    const float4 nk = *reinterpret_cast<const float4 *>(knew + (size_t)g * 256 + 4 * lane);
    const float4 nv = *reinterpret_cast<const float4 *>(vnew + (size_t)g * 256 + 4 * lane);
    // every wave's small loads enter the CU's memory pipeline before any chunk load
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    KRegs ka, kb;   // K of even / odd chunks
    VRegs va, vb;   // V of even / odd chunks
    load_k(ka, p, g, begin, 0, nchunks, length, tid);
    load_v(va, p, g, begin, 0, nchunks, tid);
    load_k(kb, p, g, begin, 1, nchunks, length, tid);
    load_v(vb, p, g, begin, 1, nchunks, tid);

    float vmax = 0.0f;
    if (p.append) {
        // the same rotation (and, for the new token, quantization) as batch_rope_int8
        // (kv_store.hip), so the cache bytes and the rotated query match it bit for bit
        const float ifreq = lane_inv_freq(p.freq);
        const Rope4 r = rope_angles(p.pos, lane, ifreq);
        const float4 z = rope4(rq, lane, r);
        if (lane < 16) *reinterpret_cast<float4 *>(&qrot0[wave][4 * lane]) = z;
        if (owner) {
            *reinterpret_cast<float4 *>(p.rotated + ((size_t)g * 8 + wave) * 256 + 4 * lane) = z;
            const uint64_t vector = (uint64_t)p.pos * 2 + g;
            if (wave == 0) {
                const float4 kz = rope4(nk, lane, r);
                const float ka = wave_max(fmaxf(fmaxf(fabsf(kz.x), fabsf(kz.y)), fmaxf(fabsf(kz.z), fabsf(kz.w))));
                const float kr127 = 127.0f / ka;
                const uint32_t codes = pack4(quant_code(kz.x, ka, kr127), quant_code(kz.y, ka, kr127),
                                             quant_code(kz.z, ka, kr127), quant_code(kz.w, ka, kr127));
                *reinterpret_cast<uint32_t *>(p.k_out + vector * 256 + 4 * lane) = codes;
                *reinterpret_cast<uint32_t *>(&fresh_k[4 * lane]) = codes;
                if (lane == 0) {
                    p.ks_out[vector] = ka / 127.0f;
                    fresh_scale[0] = ka / 127.0f;
                }
            } else if (wave == 1) {
                const float va = wave_max(fmaxf(fmaxf(fabsf(nv.x), fabsf(nv.y)), fmaxf(fabsf(nv.z), fabsf(nv.w))));
                const float vr127 = 127.0f / va;
                const float c[4] = {quant_code(nv.x, va, vr127), quant_code(nv.y, va, vr127),
                                    quant_code(nv.z, va, vr127), quant_code(nv.w, va, vr127)};
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const uint8_t b = (uint8_t)(int8_t)(int)c[i];
                    p.v_out[value_index(vector, 4 * lane + i)] = (int8_t)b;
                    fresh_v[4 * lane + i] = b;
                }
                if (lane == 0) {
                    p.vs_out[vector] = va / 127.0f;
                    fresh_scale[1] = va / 127.0f;
                }
                vmax = va / 127.0f;   // the new token joins the split's largest V scale
            }
        }
    }

    // ---- K scales of the split (this group) into LDS, vs_ref = the maximum of its V scales;
    // the per-head maxima of the query chunks
#pragma unroll
    for (int it = 0; it < kMaxSplitTokens / 512; it++) {
        const uint32_t e = tid + 512 * it;   // < kMaxSplitTokens; entries past the split are never read
        // entries past the split are zero (selected after the unconditional loads); in append
        // mode the new token's entry is set from its fresh scale below
        const bool inside = begin + e < end && (int)e != e_new;
        kscale[e] = inside ? ksv[it] * (kLog2e / 16.0f) : 0.0f;
        vmax = fmaxf(vmax, inside ? vsv[it] : 0.0f);
    }
    if (p.append) {
        __syncthreads();   // the rotated query dims and the fresh codes and scales are in LDS
        if (chunk == 0) {
            // dims 16 qq + [0, 16) of head n % 8: the rotated values
#pragma unroll
            for (int f = 0; f < 4; f++) x[f] = *reinterpret_cast<const float4 *>(&qrot0[head][16 * qq + 4 * f]);
        }
        if (tid == 0 && owner) kscale[e_new] = fresh_scale[0] * (kLog2e / 16.0f);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) vmax = fmaxf(vmax, __shfl_xor(vmax, o, 64));
    if (lane == 0) red[wave] = vmax;
    float amax = 0.0f;
#pragma unroll
    for (int f = 0; f < 4; f++) amax = fmaxf(amax, fmaxf(fmaxf(fabsf(x[f].x), fabsf(x[f].y)), fmaxf(fabsf(x[f].z), fabsf(x[f].w))));
    amax = fmaxf(amax, __shfl_xor(amax, 16, 64));
    amax = fmaxf(amax, __shfl_xor(amax, 32, 64));
    if (lane < 8 && wave < 4) qmax[wave][lane] = amax;
    __syncthreads();
    float vs_ref = red[0];
#pragma unroll
    for (int w = 1; w < kDecodeWaves; w++) vs_ref = fmaxf(vs_ref, red[w]);
    const float vs_inv = vs_ref > 0.0f ? 1.0f / vs_ref : 0.0f;
    // the split's V scales times 1 / vs_ref, the factor of the probability operand (entries past
    // the split zero, the new token's from its fresh scale); the barrier before phase 0 publishes them
#pragma unroll
    for (int it = 0; it < kMaxSplitTokens / 512; it++) {
        const uint32_t e = tid + 512 * it;
        const float s = (int)e == e_new ? fresh_scale[1] : vsv[it];
        vscale[e] = begin + e < end ? s * vs_inv : 0.0f;
    }
    // ---- INT8 query operands of chunk c = wave: q ~= s_q (q1 + q2 / 254 + q3 / 254^2).
    // z = q / s_q lies in [-127, 127]; q1 = rint(z) and r1 = z - q1 (exact, |r1| <= 1/2);
    // q2 = rint(254 r1) and r2 = 254 r1 - q2 (one rounding, |r2| <= 1/2 + 2^-17);
    // q3 = rint(254 r2). Set 0 holds q1 in columns n < 8 and q2 in n >= 8, set 1 q3 in both.
    const float qabs = fmaxf(fmaxf(qmax[0][head], qmax[1][head]), fmaxf(qmax[2][head], qmax[3][head]));
    const float qsc = qabs * (1.0f / 127.0f);   // s_q of the lane's head
    {
        const float inv = qabs > 0.0f ? 127.0f / qabs : 0.0f;
        auto code = [](float q) { return (uint32_t)(uint8_t)(int8_t)(int)fminf(fmaxf(q, -127.0f), 127.0f); };
        uint32_t w[4], w3[4];
#pragma unroll
        for (int f = 0; f < 4; f++) {
            const float xs[4] = {x[f].x, x[f].y, x[f].z, x[f].w};
            w[f] = w3[f] = 0;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const float z = xs[e] * inv, q1 = rintf(z), r1 = z - q1;
                const float q2 = rintf(r1 * 254.0f);
                const float r2 = fmaf(r1, 254.0f, -q2);
                const float q3 = rintf(r2 * 254.0f);
                w[f] |= code(lo_col ? q2 : q1) << (8 * e);
                w3[f] |= code(q3) << (8 * e);
            }
        }
        if (wave < 4) {
            qlds[0][wave][lane] = v4i{(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
            qlds[1][wave][lane] = v4i{(int)w3[0], (int)w3[1], (int)w3[2], (int)w3[3]};
        }
    }
    // K of chunk 0 into buffer 0 and K of chunk 2 into the registers it leaves
    if (jn == 0) patch_k(ka, tid, tn, reinterpret_cast<const uint4 *>(fresh_k));
    store_k(bufs[0], ka, tid);
    load_k(ka, p, g, begin, 2, nchunks, length, tid);
    __syncthreads();
    v4i qi[4], q3i[4];
#pragma unroll
    for (int c = 0; c < 4; c++) {
        qi[c] = qlds[0][c][lane];
        q3i[c] = qlds[1][c][lane];
    }

    floatx4 o[2];   // O^T tiles dt = 2 wave + i, over every token of the split
    o[0] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    o[1] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    float m = -INFINITY, l = 0.0f;

    // Probabilities of the lane's four tokens against reference ref, as the FP16 hi (column
    // n < 8) or lo (n >= 8) part of p * vs / vs_ref, published as this wave's P operand in
    // slot `slot`; total = the column's sum over the wave's 16 tokens.
    auto probs = [&](const float (&sc)[4], int local0, float ref, float &total, int slot) __attribute__((always_inline)) {
        // ref = -inf (before the first rescale) gives +inf for unmasked tokens: their chunk
        // always rescales, which rebuilds the operands and the total before either is read
        const float refc = fmaxf(ref, -3.0e38f);
        _Float16 hv[4];
        total = 0.0f;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const float prob = __builtin_amdgcn_exp2f(sc[r] - refc);   // 0 for masked tokens
            total += prob;
            const float scaled = prob * vscale[local0 + r];
            const _Float16 hi = (_Float16)scaled;
            hv[r] = lo_col ? (_Float16)(scaled - (float)hi) : hi;
        }
        total = xl_sum16(total);
        total = xl_sum32(total);
        const half4 pop = {hv[0], hv[1], hv[2], hv[3]};
        pshare[slot][wave][lane] = __builtin_bit_cast(uint2, pop);
    };
    // the previous chunk's scores, kept for a rebuild of its operands
    float sc_prev[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
    float total_prev = 0.0f;
    int local_prev = 0;
    // Phase j (one barrier each): finish chunk j - 1 (the rescale decision, then PV), score
    // chunk j, store V of chunk j and K of chunk j + 1, load V of chunk j + 2 and K of chunk
    // j + 3 into the registers just stored. K is staged one chunk ahead of V, so the two
    // buffers' K and V halves have different lifetimes: in phase j chunk j - 1's V and chunk
    // j's K are read while chunk j's V and chunk j + 1's K are written.
    // The waves share one running reference m per column; a chunk rescales (and pays a
    // second barrier) only when some column's maximum passes m by more than 2^8, so
    // p = 2^(s - m) stays below 256.
    auto finish = [&](uint32_t j) __attribute__((always_inline)) {   // chunk j - 1, j > 0
        {
            const int slot = (j - 1) & 1;
            float ctop = chunk_top[slot][0][n];
#pragma unroll
            for (int w = 1; w < kDecodeWaves; w++) ctop = fmaxf(ctop, chunk_top[slot][w][n]);
            // every wave reads the same maxima: the branch is uniform over the work-group
            if (__builtin_amdgcn_ballot_w64(ctop > m + 8.0f) != 0) {
                const float next = fmaxf(m, ctop);
                const float decay = next == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(m - next);
                l *= decay;
                o[0] *= decay;
                o[1] *= decay;
                m = next;
                probs(sc_prev, local_prev, m, total_prev, slot);   // no wave reads the slot before this branch
                __syncthreads();
            }
            l += total_prev;   // this wave's tokens
            // O^T[d][n] += V^T[d][t] P[t][n] for this wave's 32 dimensions over the chunk's 128
            // tokens on v_mfma_f32_16x16x32_f16: k-step s takes waves 2s and 2s + 1's tokens (32),
            // lane (n, qq) tokens 8 (qq % 2) .. + 7 of wave 2s + qq / 2, i.e. the published P
            // operands of lanes n + 32 (qq % 2) and n + 32 (qq % 2) + 16 of that wave and 8 codes
            // (one 8-byte read) of its V piece. Against 16 MFMAs of 16 tokens with a 4-byte read
            // each: half the MFMAs, dependent steps and V reads (29.6-30.0 against 30.2-30.3 us
            // per layer step at 131073)
            const ChunkLds &b = bufs[slot];
#pragma unroll
            for (int s = 0; s < kDecodeWaves / 2; s++) {
                const int src = 2 * s + (qq >> 1);
                const uint2 pa = pshare[slot][src][n + 32 * (qq & 1)], pb = pshare[slot][src][n + 32 * (qq & 1) + 16];
                const half8 ps = __builtin_bit_cast(half8, make_uint4(pa.x, pa.y, pb.x, pb.y));
#pragma unroll
                for (int jj = 0; jj < 2; jj++) {
                    const int d = 16 * (2 * wave + jj) + n;
                    const uint2 w8 = reinterpret_cast<const uint2 *>(&b.v[d][src ^ ((d >> 1) & 7)])[qq & 1];
                    uint32_t h0, h1, h2, h3;
                    i8x8_to_f16_sdwa(w8.x, w8.y, h0, h1, h2, h3);
                    const half8 va8 = __builtin_bit_cast(half8, make_uint4(h0, h1, h2, h3));
                    o[jj] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va8, ps, o[jj], 0, 0, 0);
                }
            }
        }
    };
    // odd: a compile-time parity of j, which picks the register sets (V of chunk j, K of
    // chunk j + 1) without taking their addresses
    auto phase = [&](uint32_t j, auto odd, bool store_knext, bool load_v2, bool load_k3) __attribute__((always_inline)) {
        VRegs &rv = decltype(odd)::value ? vb : va;
        KRegs &rk = decltype(odd)::value ? ka : kb;
        if (j > 0) finish(j);
        {
            const ChunkLds &b = bufs[j & 1];
            const int tl = 16 * wave + (lane & 15);          // the lane's K row of the chunk
            // S^T: rows = tokens 16w + 4qq + r of the chunk, columns n; acc3 holds the q3 part
            v4i acc = {0, 0, 0, 0}, acc3 = {0, 0, 0, 0};
#pragma unroll
            for (int jj = 0; jj < 4; jj++) {
                const v4i kop = __builtin_bit_cast(v4i, b.k[tl][(4 * jj + qq) ^ (tl & 15)]);
                acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(kop, qi[jj], acc, 0, 0, 0);
                acc3 = __builtin_amdgcn_mfma_i32_16x16x64_i8(kop, q3i[jj], acc3, 0, 0, 0);
            }
            // the partner column n ^ 8 holds the other part of the same head; every dot is
            // an integer below 2^22 in magnitude, exact in FP32
            const int local0 = (int)(j * kChunk) + 16 * wave + 4 * qq;   // token offset inside the split
            const uint32_t t0 = begin + (uint32_t)local0;
            float top = -INFINITY;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const float mine = (float)acc[r], other = xl_swap8(mine);   // exact: |dot| < 2^22
                const float hi = lo_col ? other : mine, lo = lo_col ? mine : other;
                const float full = fmaf((float)acc3[r], 1.0f / 64516.0f, fmaf(lo, 1.0f / 254.0f, hi)) * qsc;
                const float value = t0 + r < end ? full * kscale[local0 + r] : -INFINITY;
                sc_prev[r] = value;
                top = fmaxf(top, value);
            }
            top = xl_max16(top);
            top = xl_max32(top);
            local_prev = local0;
            probs(sc_prev, local0, m, total_prev, j & 1);
            if (qq == 0) chunk_top[j & 1][wave][n] = top;
        }
        if ((int)j == jn) patch_v(rv, tid, tn, fresh_v);
        store_v(bufs[j & 1], rv, tid);
        if (load_v2) load_v(rv, p, g, begin, j + 2, nchunks, tid);
        if ((int)j + 1 == jn) patch_k(rk, tid, tn, reinterpret_cast<const uint4 *>(fresh_k));
        if (store_knext) store_k(bufs[(j + 1) & 1], rk, tid);
        if (load_k3) load_k(rk, p, g, begin, j + 3, nchunks, length, tid);
        __syncthreads();
    };
    // Phases in pairs, so that the register sets keep fixed roles without copies (a copy of
    // registers still being loaded waits for the load). The pairs run while every load is
    // a real chunk (a fixed count per pair keeps the counter waits exact); the last one to
    // four chunks follow without loads past the end, whose registers the end of the
    // work-group would otherwise wait for.
    uint32_t c = 0;
    for (; c + 4 < nchunks; c += 2) {
        phase(c, std::false_type{}, true, true, true);
        phase(c + 1, std::true_type{}, true, true, true);
    }
    if (c < nchunks) {
        phase(c, std::false_type{}, c + 1 < nchunks, c + 2 < nchunks, c + 3 < nchunks);
        uint32_t last_phase = c + 1;
        if (c + 1 < nchunks) {
            phase(c + 1, std::true_type{}, c + 2 < nchunks, c + 3 < nchunks, false);
            last_phase = c + 2;
            if (c + 2 < nchunks) {
                phase(c + 2, std::false_type{}, c + 3 < nchunks, false, false);
                last_phase = c + 3;
                if (c + 3 < nchunks) {
                    phase(c + 3, std::true_type{}, false, false, false);
                    last_phase = c + 4;
                }
            }
        }
        finish(last_phase);
    }

    // ---- the waves share m; l sums over waves. O^T[d][n], d = 16 dt + 4 qq + r: the lo
    // column n + 8 of each head joins its hi column n in registers (the DPP adds take MFMA
    // results as inline-assembly operands, for which the compiler inserts no wait states:
    // cover them here), then lanes n < 8 hold tile 2 wave and lanes n >= 8 tile 2 wave + 1.
    if (qq == 0) wave_l[wave][n] = l;
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7");
    __builtin_amdgcn_sched_barrier(0);
    add_row_partner8(o[0], o[1]);
    __syncthreads();
    float lw = 0.0f;
#pragma unroll
    for (int w = 0; w < kDecodeWaves; w++) lw += wave_l[w][head];
    const bool upper = n >= 8;
    const int d0 = 16 * (2 * wave + (upper ? 1 : 0)) + 4 * qq;
    const int h = head;
    const float mw = m;
    floatx4 res = upper ? o[1] : o[0];
    float4 acc = make_float4(res[0] * vs_ref, res[1] * vs_ref, res[2] * vs_ref, res[3] * vs_ref);
    if (p.splits == 1) {
        // gate and y need only 4-byte alignment
        // (the four gate loads go out before the first store: the compiler cannot tell y from gate)
        const size_t at = ((size_t)row * 16 + g * 8 + h) * 256 + d0;
        const float inv = 1.0f / lw;
        const float g0 = p.gate[at + 0], g1 = p.gate[at + 1], g2 = p.gate[at + 2], g3 = p.gate[at + 3];
        asm volatile("" ::"v"(g0), "v"(g1), "v"(g2), "v"(g3) : "memory");
        p.y[at + 0] = acc.x * inv * sigmoidf(g0);
        p.y[at + 1] = acc.y * inv * sigmoidf(g1);
        p.y[at + 2] = acc.z * inv * sigmoidf(g2);
        p.y[at + 3] = acc.w * inv * sigmoidf(g3);
        return;
    }
    float *part = p.partial + (((size_t)row * 2 + g) * p.splits + split) * kPartialFloats;
    *reinterpret_cast<float4 *>(part + h * 256 + d0) = acc;
    if (wave == 0 && lane < 8) {
        part[2048 + h] = mw;
        part[2056 + h] = lw;
    }
}

// Merges the splits of one (row, head) (grid: 4 x 16 heads x rows, four waves per work-group).
// Each wave owns 16 dimensions and works alone (no LDS, no barrier): lane (sg, q) holds the
// float4 of dimensions 4q .. 4q + 3 for splits sg, sg + 16, ... (the first 128 splits' m, l and
// partials loaded at once), the maximum of m and then the weighted sums of l and O are reduced
// over the 16 split groups, and the lanes of group 0 write the output. The order of every sum
// is fixed by the split count alone.
__global__ __launch_bounds__(256) void decode_combine_kernel(const float *__restrict__ partial, const float *__restrict__ gate,
                                                             float *__restrict__ y, uint32_t splits) {
    const uint32_t row = blockIdx.z, hq = blockIdx.y, g = hq / 8, h = hq % 8;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int q = lane & 3, sg = lane >> 2;
    const uint32_t d = (blockIdx.x * 4 + wave) * 16 + 4 * q;
    const float *base = partial + ((size_t)row * 2 + g) * splits * kPartialFloats;
    constexpr int kEarly = 8;
    float mv[kEarly], lv[kEarly];
    float4 ov[kEarly];
#pragma unroll
    for (int u = 0; u < kEarly; u++) {
        const uint32_t s = sg + 16 * u, sidx = min(s, splits - 1);
        const float *sp = base + (size_t)sidx * kPartialFloats;
        ov[u] = *reinterpret_cast<const float4 *>(sp + h * 256 + d);
        mv[u] = s < splits ? sp[2048 + h] : -INFINITY;
        lv[u] = sp[2056 + h];
    }
    const size_t at = ((size_t)row * 16 + hq) * 256 + d;
    float gv[4];
#pragma unroll
    for (int i = 0; i < 4; i++) gv[i] = gate[at + i];   // y and gate need only 4-byte alignment
    float mmax = mv[0];
#pragma unroll
    for (int u = 1; u < kEarly; u++) mmax = fmaxf(mmax, mv[u]);
    for (uint32_t s = sg + 16 * kEarly; s < splits; s += 16) mmax = fmaxf(mmax, base[(size_t)s * kPartialFloats + 2048 + h]);
#pragma unroll
    for (int o = 4; o < 64; o <<= 1) mmax = fmaxf(mmax, __shfl_xor(mmax, o, 64));
    float lsum = 0.0f;
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    auto add = [&](float m, float l, const float4 &o) {
        if (m == -INFINITY) return;   // a split that holds none of the row's keys
        const float w = __builtin_amdgcn_exp2f(m - mmax);
        lsum += l * w;
        acc.x += o.x * w;
        acc.y += o.y * w;
        acc.z += o.z * w;
        acc.w += o.w * w;
    };
#pragma unroll
    for (int u = 0; u < kEarly; u++) add(mv[u], lv[u], ov[u]);
    for (uint32_t s = sg + 16 * kEarly; s < splits; s += 16) {
        const float *sp = base + (size_t)s * kPartialFloats;
        add(sp[2048 + h], sp[2056 + h], *reinterpret_cast<const float4 *>(sp + h * 256 + d));
    }
#pragma unroll
    for (int o = 4; o < 64; o <<= 1) {
        lsum += __shfl_xor(lsum, o, 64);
        acc.x += __shfl_xor(acc.x, o, 64);
        acc.y += __shfl_xor(acc.y, o, 64);
        acc.z += __shfl_xor(acc.z, o, 64);
        acc.w += __shfl_xor(acc.w, o, 64);
    }
    if (sg == 0) {
        const float inv = 1.0f / lsum;
        y[at + 0] = acc.x * inv * sigmoidf(gv[0]);
        y[at + 1] = acc.y * inv * sigmoidf(gv[1]);
        y[at + 2] = acc.z * inv * sigmoidf(gv[2]);
        y[at + 3] = acc.w * inv * sigmoidf(gv[3]);
    }
}

inline bool aligned(const void *p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

}  // namespace

const char *launch_scores_int8(Context &c, const View *b, int count, const boot_kernel_args &p, const uint32_t *) {
    // bindings: q FP32 [rows][16][256], k INT8 cache, scores [rows][16][K], ks (QwenEngine.cs:163, Prefill.cs:280)
    BOOT_REQUIRE(count >= 4, "batch_attention_scores_int8 needs 4 bindings: q, k, scores, ks");
    const uint64_t rows = p.m, K = p.k;
    if (rows == 0 || K == 0) return nullptr;
    const uint64_t length = std::min<uint64_t>(K, (uint64_t)p.pos + rows);  // keys actually read
    BOOT_REQUIRE(b[0].bytes >= rows * 16384, "query buffer smaller than rows*4096 floats");
    BOOT_REQUIRE(b[1].bytes >= length * 512, "K cache smaller than the attended length");
    BOOT_REQUIRE(b[2].bytes >= rows * 16 * K * 4, "scores buffer smaller than rows*16*K floats");
    BOOT_REQUIRE(b[3].bytes >= length * 8, "K scale buffer smaller than the attended length");
    BOOT_REQUIRE(aligned(b[0].ptr, 4) && aligned(b[1].ptr, 16) && aligned(b[2].ptr, 4) && aligned(b[3].ptr, 4),
                 "bindings misaligned");
    // rows per work-group: the fewest of 1, 2, 4 that hold the dispatch's rows, at most 4 (an
    // 8-row work-group reads K once for all rows but holds one work-group per CU and streams
    // slower: 63.6 against 54.0 us at 8 rows over 131072 keys); a row's scores are the same in each
    const int per = rows >= 3 ? 4 : rows == 2 ? 2 : 1;
    const uint64_t zs = (rows + per - 1) / per;
    BOOT_REQUIRE(zs <= 65535, "batch_attention_scores_int8 serves at most 262140 rows");
    // tokens per work-group: 512 where the grid still holds four work-groups per CU (each one then
    // builds its rows' query operands for twice the tokens: 8 rows over 131072 keys 38.3 -> 32.7
    // us), else 256 (4 rows over 30000 keys: 12.5 us, against 18.1 with 512); a score does not
    // depend on the span
    const uint64_t wide = (K + 511) / 512;
    const uint32_t span = 2 * wide * zs >= 4 * (uint64_t)std::max(1, context_cus(c)) ? 512u : 256u;
    const uint64_t ktiles = (K + span - 1) / span;
    const dim3 sgrid((uint32_t)((2 * ktiles + 7) / 8 * 8 * zs));
    const float *qp = (const float *)b[0].ptr, *ksp = (const float *)b[3].ptr;
    const int8_t *kp = (const int8_t *)b[1].ptr;
    float *sp = (float *)b[2].ptr;
    if (per == 4)
        launch_timed(c, "scores_int8_kernel", scores_int8_kernel<4>, sgrid, dim3(256), qp, kp, sp, ksp, (uint32_t)rows,
                     (uint32_t)K, p.pos, (uint32_t)ktiles, (uint32_t)zs, span);
    else if (per == 2)
        launch_timed(c, "scores_int8_kernel", scores_int8_kernel<2>, sgrid, dim3(256), qp, kp, sp, ksp, (uint32_t)rows,
                     (uint32_t)K, p.pos, (uint32_t)ktiles, (uint32_t)zs, span);
    else
        launch_timed(c, "scores_int8_kernel", scores_int8_kernel<1>, sgrid, dim3(256), qp, kp, sp, ksp, (uint32_t)rows,
                     (uint32_t)K, p.pos, (uint32_t)ktiles, (uint32_t)zs, span);
    return nullptr;
}

const char *launch_softmax(Context &c, const View *b, int count, const boot_kernel_args &p, const uint32_t *grid) {
    // bindings: x scores [groups][K]; groups = dispatched threads / 256 (QwenEngine.cs:164, Prefill.cs:282)
    BOOT_REQUIRE(count >= 1, "attention_softmax needs 1 binding: scores");
    BOOT_REQUIRE(grid[3] == 256 && grid[1] <= 1 && grid[2] <= 1, "attention_softmax is dispatched as groups of 256 threads");
    const uint64_t groups = grid[0] / 256, K = p.k;
    if (groups == 0) return nullptr;
    BOOT_REQUIRE(p.pos < K, "softmax position must be below the row stride K");
    BOOT_REQUIRE(b[0].bytes >= groups * K * 4, "scores buffer smaller than groups*K floats");
    BOOT_REQUIRE(aligned(b[0].ptr, 4), "scores binding misaligned");
    // chunk statistics of every row, then each chunk normalized with its row's merged statistics
    const uint64_t chunks = ((uint64_t)p.pos + 1 + kSoftmaxChunk - 1) / kSoftmaxChunk;
    BOOT_REQUIRE(groups <= 65535, "attention_softmax serves at most 65535 rows");
    float2 *stats = (float2 *)context_workspace(c, groups * chunks * sizeof(float2));
    BOOT_REQUIRE(stats, "cannot allocate softmax workspace");
    const dim3 sgrid((uint32_t)chunks, (uint32_t)groups);
    launch_timed(c, "softmax_stats_kernel", softmax_stats_kernel, sgrid, dim3(256), (const float *)b[0].ptr, stats,
                 (uint32_t)K, p.pos, (uint32_t)chunks);
    launch_timed(c, "softmax_apply_kernel", softmax_apply_kernel, sgrid, dim3(256), (float *)b[0].ptr,
                 (const float2 *)stats, (uint32_t)K, p.pos, (uint32_t)chunks);
    return nullptr;
}

const char *launch_values_int8(Context &c, const View *b, int count, const boot_kernel_args &p, const uint32_t *) {
    // bindings: scores, v INT8 pages, gate, y, vs (QwenEngine.cs:165, Prefill.cs:283)
    BOOT_REQUIRE(count >= 5, "batch_attention_values_int8 needs 5 bindings: scores, v, gate, y, vs");
    const uint64_t rows = p.m, K = p.k;
    if (rows == 0) return nullptr;
    BOOT_REQUIRE(rows <= 65535, "batch_attention_values_int8 serves at most 65535 rows");   // the combine's grid
    const uint64_t length = (uint64_t)p.pos + rows;
    BOOT_REQUIRE(length <= K, "causal end pos+rows exceeds the score row stride K");
    BOOT_REQUIRE(b[0].bytes >= rows * 16 * K * 4, "scores buffer smaller than rows*16*K floats");
    BOOT_REQUIRE(b[1].bytes >= value_bytes(length), "V cache smaller than whole pages of the attended length");
    BOOT_REQUIRE(b[2].bytes >= rows * 16384 && b[3].bytes >= rows * 16384, "gate/output smaller than rows*4096 floats");
    BOOT_REQUIRE(b[4].bytes >= length * 8, "V scale buffer smaller than the attended length");
    BOOT_REQUIRE(aligned(b[1].ptr, 16), "V cache binding must be 16-byte aligned");
    // split partials over absolute kValuesSplit-token ranges, then their sum in order with the gate
    const uint64_t splits = (K + kValuesSplit - 1) / kValuesSplit;
    float *part = (float *)context_workspace(c, rows * 2 * splits * 2048 * sizeof(float));
    BOOT_REQUIRE(part, "cannot allocate values workspace");
    // rows per work-group: the fewest of 1, 2, 4 that hold the dispatch's rows, at most 4 (8 rows
    // take 276 registers, one work-group per CU: 74.0 against 52.2 us at 8 rows over 131072 keys;
    // 2 rows read V four times: 63.6 us); a row's result is the same in each
    const int per = rows >= 3 ? 4 : rows == 2 ? 2 : 1;
    const uint64_t zs = (rows + per - 1) / per;
    const dim3 vgrid((uint32_t)((2 * splits + 7) / 8 * 8 * zs));
    const float *sc = (const float *)b[0].ptr, *vsc = (const float *)b[4].ptr;
    const int8_t *vc = (const int8_t *)b[1].ptr;
    if (per == 4)
        launch_timed(c, "values_partial_kernel", values_partial_kernel<4>, vgrid, dim3(512), sc, vc, vsc, part,
                     (uint32_t)rows, (uint32_t)K, p.pos, (uint32_t)splits, (uint32_t)zs);
    else if (per == 2)
        launch_timed(c, "values_partial_kernel", values_partial_kernel<2>, vgrid, dim3(512), sc, vc, vsc, part,
                     (uint32_t)rows, (uint32_t)K, p.pos, (uint32_t)splits, (uint32_t)zs);
    else
        launch_timed(c, "values_partial_kernel", values_partial_kernel<1>, vgrid, dim3(512), sc, vc, vsc, part,
                     (uint32_t)rows, (uint32_t)K, p.pos, (uint32_t)splits, (uint32_t)zs);
    launch_timed(c, "values_combine_kernel", values_combine_kernel, dim3(64, (uint32_t)rows), dim3(64),
                 (const float *)part, (const float *)b[2].ptr, (float *)b[3].ptr, (uint32_t)splits);
    return nullptr;
}

namespace {

// Split geometry shared by both decode entry points: whole 128-token chunks per split, chosen so
// that the grid (splits x 2 groups x rows, one work-group per CU) fits the CUs in one round (a
// second, nearly empty round would double the time), at most kMaxSplitTokens per split.
template <bool kHalfQ = false>
const char *decode_launch(Context &c, DecodeParams &d, uint64_t rows, uint64_t length) {
    const uint64_t total_chunks = (length + kChunk - 1) / kChunk;
    const uint64_t slots = std::max<uint64_t>(1, (uint64_t)std::max(1, context_cus(c)) / (2 * rows));
    uint64_t split_chunks = (total_chunks + slots - 1) / slots;
    split_chunks = std::min<uint64_t>(split_chunks, (uint64_t)(kMaxSplitTokens / kChunk));
    const uint64_t splits = (total_chunks + split_chunks - 1) / split_chunks;
    BOOT_REQUIRE(splits <= kMaxDecodeSplits, "too many decode splits");
    d.rows = (uint32_t)rows;
    d.splits = (uint32_t)splits;
    d.split_chunks = (uint32_t)split_chunks;
    d.partial = nullptr;
    if (splits > 1) {
        d.partial = (float *)context_workspace(c, rows * 2 * splits * kPartialFloats * sizeof(float));
        BOOT_REQUIRE(d.partial, "cannot allocate decode split workspace");
    }
    launch_timed(c, kHalfQ ? "decode_int8_half_query_kernel" : "decode_int8_kernel", decode_int8_kernel<kHalfQ>,
                 dim3((uint32_t)splits, 2, (uint32_t)rows), dim3(512), d);
    if (splits > 1) {
        context_split(c, "attention_decode_int8.combine");
        launch_timed(c, "decode_combine_kernel", decode_combine_kernel, dim3(4, 16, (uint32_t)rows), dim3(256), d.partial,
                     d.gate, d.y, (uint32_t)splits);
    }
    return nullptr;
}

}  // namespace

const char *launch_decode_append_int8(Context &c, const View *b, int count, const boot_kernel_args &p,
                                      const uint32_t *) {
    // bindings: q FP32 [1][16][256] (unrotated), k, v FP32 [1][2][256] (the new token, K
    // unrotated), rotated FP32 [1][16][256] (out), kc, vc, ks, vs (the cache, appended at
    // Position), gate, y. One decode step of QwenEngine.cs:161-165: batch_rope_int8 with M = 1
    // followed by attention over keys 0..Position, in one dispatch.
    BOOT_REQUIRE(count >= 10, "attention_decode_append_int8 needs 10 bindings: q, k, v, rotated, kc, vc, ks, vs, gate, y");
    BOOT_REQUIRE(p.m == 1, "attention_decode_append_int8 serves one row (M = 1)");
    const uint64_t length = (uint64_t)p.pos + 1;
    BOOT_REQUIRE(length <= 262144, "attended length exceeds the 262144-token window");
    BOOT_REQUIRE(b[0].bytes >= 16384 && b[3].bytes >= 16384, "query/rotated buffers smaller than 4096 floats");
    BOOT_REQUIRE(b[1].bytes >= 2048 && b[2].bytes >= 2048, "K/V input smaller than 512 floats");
    BOOT_REQUIRE(b[4].bytes >= length * 512, "K cache smaller than Position + 1 tokens");
    BOOT_REQUIRE(b[5].bytes >= value_bytes(length), "V cache smaller than whole pages of Position + 1 tokens");
    BOOT_REQUIRE(b[6].bytes >= length * 8 && b[7].bytes >= length * 8, "KV scale buffers smaller than Position + 1 tokens");
    BOOT_REQUIRE(b[8].bytes >= 16384 && b[9].bytes >= 16384, "gate/output smaller than 4096 floats");
    BOOT_REQUIRE(aligned(b[0].ptr, 16) && aligned(b[1].ptr, 16) && aligned(b[2].ptr, 16) && aligned(b[3].ptr, 16) &&
                     aligned(b[4].ptr, 16) && aligned(b[5].ptr, 16) && aligned(b[6].ptr, 4) && aligned(b[7].ptr, 4) &&
                     aligned(b[8].ptr, 4) && aligned(b[9].ptr, 4),
                 "bindings misaligned (q, k, v, rotated, kc, vc need 16 bytes)");
    DecodeParams d;
    d.q = (const float *)b[0].ptr;
    d.qh = nullptr;
    d.knew = (const float *)b[1].ptr;
    d.vnew = (const float *)b[2].ptr;
    d.rotated = (float *)b[3].ptr;
    d.k = (const int8_t *)b[4].ptr;
    d.v = (const int8_t *)b[5].ptr;
    d.ks = (const float *)b[6].ptr;
    d.vs = (const float *)b[7].ptr;
    d.k_out = (int8_t *)b[4].ptr;
    d.v_out = (int8_t *)b[5].ptr;
    d.ks_out = (float *)b[6].ptr;
    d.vs_out = (float *)b[7].ptr;
    d.gate = (const float *)b[8].ptr;
    d.y = (float *)b[9].ptr;
    d.pos = p.pos;
    d.append = 1;
    d.freq = rope_frequencies(p.theta);
    return decode_launch(c, d, 1, length);
}

const char *launch_decode_int8(Context &c, const View *b, int count, const boot_kernel_args &p, const uint32_t *) {
    // bindings (EncodeInt8 order, DeviceAttention.cs:69): q FP32 [rows][16][256] (rotated),
    // k, v, gate, y, ks, vs. Row r attends t <= pos + r.
    BOOT_REQUIRE(count >= 7, "attention_decode_int8 needs 7 bindings: q, k, v, gate, y, ks, vs");
    const uint64_t rows = p.m;
    if (rows == 0) return nullptr;
    BOOT_REQUIRE(rows <= 64, "attention_decode_int8 serves at most 64 rows");
    const uint64_t length = (uint64_t)p.pos + rows;
    BOOT_REQUIRE(length <= 262144, "attended length exceeds the 262144-token window");
    BOOT_REQUIRE(b[0].bytes >= rows * 16384, "query buffer smaller than rows*4096 floats");
    BOOT_REQUIRE(b[1].bytes >= length * 512, "K cache smaller than the attended length");
    BOOT_REQUIRE(b[2].bytes >= value_bytes(length), "V cache smaller than whole pages of the attended length");
    BOOT_REQUIRE(b[3].bytes >= rows * 16384 && b[4].bytes >= rows * 16384, "gate/output smaller than rows*4096 floats");
    BOOT_REQUIRE(b[5].bytes >= length * 8 && b[6].bytes >= length * 8, "KV scale buffers smaller than the attended length");
    BOOT_REQUIRE(aligned(b[0].ptr, 16) && aligned(b[1].ptr, 16) && aligned(b[2].ptr, 16) && aligned(b[3].ptr, 4) &&
                     aligned(b[4].ptr, 4) && aligned(b[5].ptr, 4) && aligned(b[6].ptr, 4),
                 "bindings misaligned (q, k, v need 16 bytes)");
    DecodeParams d;
    d.q = (const float *)b[0].ptr;
    d.qh = nullptr;
    d.k = (const int8_t *)b[1].ptr;
    d.v = (const int8_t *)b[2].ptr;
    d.gate = (const float *)b[3].ptr;
    d.y = (float *)b[4].ptr;
    d.ks = (const float *)b[5].ptr;
    d.vs = (const float *)b[6].ptr;
    d.pos = p.pos;
    d.append = 0;
    d.freq = RopeFreq{};
    d.knew = d.vnew = nullptr;
    d.rotated = nullptr;
    d.k_out = d.v_out = nullptr;
    d.ks_out = d.vs_out = nullptr;
    return decode_launch(c, d, rows, length);
}

const char *launch_online_int8_as_decode(Context &c, const View *b, const boot_kernel_args &p) {
    // A prefill chunk of at most 64 rows over a short history (launch_prefill's choice, which has
    // validated the bindings: grouped FP16 q, k, v, gate, y, ks, vs): one work-group per (row, KV
    // group, split) streams the keys up to its own row's position, as a decode of that many rows,
    // instead of 256-row tiles that are mostly empty.
    const uint64_t rows = p.m, length = (uint64_t)p.pos + rows;
    BOOT_REQUIRE(rows >= 1 && rows <= 64, "a prefill chunk served by the decode kernel has 1 to 64 rows");
    DecodeParams d;
    d.q = nullptr;
    d.qh = (const _Float16 *)b[0].ptr;
    d.k = (const int8_t *)b[1].ptr;
    d.v = (const int8_t *)b[2].ptr;
    d.gate = (const float *)b[3].ptr;
    d.y = (float *)b[4].ptr;
    d.ks = (const float *)b[5].ptr;
    d.vs = (const float *)b[6].ptr;
    d.pos = p.pos;
    d.append = 0;
    d.freq = RopeFreq{};
    d.knew = d.vnew = nullptr;
    d.rotated = nullptr;
    d.k_out = d.v_out = nullptr;
    d.ks_out = d.vs_out = nullptr;
    return decode_launch<true>(c, d, rows, length);
}

}  // namespace boot
