// Single-token (and 1-8 row verification) INT8 attention over the KV cache.
//
// Two entry points:
//   * the reference's three-kernel reader (kernels.metal:147-156,163-166):
//     batch_attention_scores_int8 -> attention_softmax -> batch_attention_values_int8,
//     FP32 scores in a caller buffer; serves serial decode and speculative
//     verification unchanged (QwenEngine.cs:161-165, Prefill.cs:280-285).
//   * attention_decode_int8: one fused split-K pass that streams the INT8 K/V
//     pages from HBM once. Scores run on INT8 MFMA straight from the K codes:
//     the FP32 query of each head is split into two INT8 parts,
//     q ~= s_q (q1 + q2 / 254) with s_q = max|q| / 127 (error <= 1.55e-5 max|q|),
//     which fill the 16 MFMA columns (8 heads x {q1, q2}). PV runs on FP16 MFMA
//     with V codes dequantized exactly in registers and the scaled
//     probabilities p*vs[t]/vs_ref (vs_ref = the largest V scale of the split, so
//     they lie in [0, 1]) split into FP16 hi + lo. Scales are applied to scores
//     and probabilities as the reference does (score = dot * ks[t] / 16,
//     P = p * vs[t]).
#include "common.h"
#include "mfma.h"

namespace boot {


namespace {

// ---------------------------------------------------------------- reference-compatible reader

// scores[(row*16+h)*K + t] = (q . code) * ks[t*2+h/8] * (1/16), -inf beyond row's
// causal end (kernels.metal:147-152). One thread per token, eight heads of one
// KV group per block.
__global__ __launch_bounds__(64) void scores_int8_kernel(const float *__restrict__ q, const int8_t *__restrict__ k,
                                                         float *__restrict__ scores, const float *__restrict__ ks,
                                                         uint32_t rows, uint32_t K, uint32_t pos) {
    __shared__ float qs[8][256];
    const uint32_t row = blockIdx.y >> 1, g = blockIdx.y & 1;
    for (int i = threadIdx.x; i < 8 * 256; i += 64) qs[i / 256][i % 256] = q[(size_t)row * 4096 + (g * 8) * 256 + i];
    __syncthreads();
    const uint32_t t = blockIdx.x * 64 + threadIdx.x;
    if (t >= K) return;
    float acc[8];
    const bool visible = t <= pos + row;
    if (visible) {
#pragma unroll
        for (int h = 0; h < 8; h++) acc[h] = 0.0f;
        const int8_t *kr = k + ((size_t)t * 2 + g) * 256;
        for (int d0 = 0; d0 < 256; d0 += 16) {
            const uint4 w = *reinterpret_cast<const uint4 *>(kr + d0);
            const uint32_t words[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
            for (int j = 0; j < 16; j++) {
                const float code = (float)(int8_t)((words[j >> 2] >> (8 * (j & 3))) & 0xff);
#pragma unroll
                for (int h = 0; h < 8; h++) acc[h] = fmaf(qs[h][d0 + j], code, acc[h]);
            }
        }
    }
    const float scale = visible ? ks[(size_t)t * 2 + g] : 0.0f;
#pragma unroll
    for (int h = 0; h < 8; h++)
        scores[((size_t)row * 16 + g * 8 + h) * K + t] = visible ? acc[h] * scale * (1.0f / 16.0f) : -INFINITY;
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

// In-place three-pass softmax over i <= pos of each row (kernels.metal:163-166).
__global__ __launch_bounds__(256) void softmax_kernel(float *__restrict__ x, uint32_t K, uint32_t pos) {
    __shared__ float partial[4];
    float *r = x + (size_t)blockIdx.x * K;
    float top = -INFINITY;
    for (uint32_t i = threadIdx.x; i <= pos; i += 256) top = fmaxf(top, r[i]);
    top = block_reduce_256(top, partial, true);
    float sum = 0.0f;
    for (uint32_t i = threadIdx.x; i <= pos; i += 256) {
        const float value = expf(r[i] - top);
        r[i] = value;
        sum += value;
    }
    sum = block_reduce_256(sum, partial, false);
    for (uint32_t i = threadIdx.x; i <= pos; i += 256) r[i] /= sum;
}

// y[(row*16+h)*256+d] = sum_t scores*vs*vcode * sigmoid(gate) (kernels.metal:153-156).
__global__ __launch_bounds__(256) void values_int8_kernel(const float *__restrict__ scores, const int8_t *__restrict__ v,
                                                          const float *__restrict__ gate, float *__restrict__ y,
                                                          const float *__restrict__ vs, uint32_t rows, uint32_t K,
                                                          uint32_t pos) {
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i >= rows * 4096) return;
    const uint32_t row = i / 4096, h = (i % 4096) / 256, d = i % 256, g = h / 8;
    const float *s = scores + ((size_t)row * 16 + h) * K;
    const uint32_t end = pos + row + 1;
    float sum = 0.0f;
    uint32_t t = 0;
    for (; t + 16 <= end && ((t & 255) + 16 <= 256); t += 16) {
        const uint4 w = *reinterpret_cast<const uint4 *>(v + value_index((uint64_t)t * 2 + g, d));
        const uint32_t words[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int j = 0; j < 16; j++) {
            const float code = (float)(int8_t)((words[j >> 2] >> (8 * (j & 3))) & 0xff);
            sum += s[t + j] * vs[(size_t)(t + j) * 2 + g] * code;
        }
    }
    for (; t < end; t++) sum += s[t] * vs[(size_t)t * 2 + g] * (float)v[value_index((uint64_t)t * 2 + g, d)];
    y[i] = sum * (1.0f / (1.0f + expf(-gate[i])));
}

// ---------------------------------------------------------------- fused split-K decode

constexpr int kDecodeBlock = 32;                 // tokens per MFMA block
constexpr int kDecodeWaves = 4;
constexpr int kMaxSplitTokens = 2048;            // tokens per work-group at most (LDS scales)
constexpr int kPartialFloats = 8 * 256 + 16;    // O[8][256], m[8], l[8] per (row, group, split)
constexpr int kMaxDecodeSplits = 1024;
constexpr float kLog2e = 1.4426950408889634f;

struct DecodeParams {
    const float *q;
    const int8_t *k;
    const int8_t *v;
    const float *ks;
    const float *vs;
    const float *gate;
    float *y;
    float *partial;
    uint32_t rows, pos, splits;
    uint32_t split_blocks;   // 32-token blocks per split
};

__device__ inline float sigmoidf(float x) { return 1.0f / (1.0f + expf(-x)); }

struct DecodeBlock {
    uint4 k[2][4];    // K tiles a = 0, 1: 16 codes at dims 16*qq + 64*j of this lane's token
    uint2 v[16];      // V^T rows d = 16*dt + n: 8 codes of tokens t0 + 8*qq + [0, 8)
};

// K tile a row i holds token t0 + 8*(i/4) + 4*a + i%4, so after the QK MFMA lane
// group qq owns tokens t0 + 8*qq + [0, 8), the k-group of the PV MFMA. Addresses
// are clamped inside the cache; tokens at or beyond the split end are masked.
__device__ inline void load_block(DecodeBlock &blk, const DecodeParams &p, uint32_t g, uint32_t t0, uint32_t length,
                                  int lane, int n, int qq) {
#pragma unroll
    for (int a = 0; a < 2; a++) {
        const uint32_t i = lane & 15;
        const uint32_t t = min(t0 + 8 * (i >> 2) + 4 * a + (i & 3), length - 1);
        const int8_t *kr = p.k + ((size_t)t * 2 + g) * 256 + 16 * qq;
#pragma unroll
        for (int j = 0; j < 4; j++) blk.k[a][j] = *reinterpret_cast<const uint4 *>(kr + 64 * j);
    }
    const uint32_t tv = min(t0 + 8 * qq, length - 1) & ~7u;
    const int8_t *vbase = p.v + value_index((uint64_t)tv * 2 + g, 0) + (size_t)n * 256;
#pragma unroll
    for (int dt = 0; dt < 16; dt++) blk.v[dt] = *reinterpret_cast<const uint2 *>(vbase + (size_t)dt * 16 * 256);
}

// Grid: (splits, 2 KV groups, rows). A split is split_blocks blocks of 32 tokens
// (chosen on the host so that the grid fits the CUs in one round); wave w takes
// blocks w, w+4, w+8, ... so the four waves consume each 128-byte V page-row
// line (128 tokens) together and lines are fetched once. Each wave walks its
// blocks with the loads of the next block in flight while the current one is
// computed. Per block: S^T[t][n] = K[t] . Qx[n] (16x16x64 INT8 MFMA on the raw K
// codes, n = 8 heads x {q1, q2}), the online softmax of the 8 heads in base 2,
// and O^T[d][n] += V^T[d][t] . Px[t][n] (16x16x32 FP16 MFMA) with
// Px = p * vs / vs_ref split into FP16 hi + lo; vs_ref, the split's largest V
// scale, keeps Px in [0, 1] and multiplies the result once.
// Lane l holds MFMA column n = l % 16 and token/k group qq = l / 16.
__global__ __launch_bounds__(256, 2) void decode_int8_kernel(DecodeParams p) {
    typedef int v4i __attribute__((ext_vector_type(4)));
    __shared__ float merge_o[kDecodeWaves][8][256];
    __shared__ float merge_m[kDecodeWaves][8], merge_l[kDecodeWaves][8];
    __shared__ float kscale[kMaxSplitTokens], vscale[kMaxSplitTokens];
    __shared__ float red[kDecodeWaves], qmax[kDecodeWaves][8];
    __shared__ v4i qlds[4][64];    // INT8 query operands, [MFMA c][lane]
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n = lane & 15, qq = lane >> 4, head = n & 7;
    const bool lo_col = n >= 8;
    const uint32_t split = blockIdx.x, g = blockIdx.y, row = blockIdx.z;
    const uint32_t length = p.pos + row + 1;
    const uint32_t split_tokens = p.split_blocks * kDecodeBlock;
    const uint32_t begin = split * split_tokens;
    const uint32_t end = min(length, begin + split_tokens);
    const uint32_t nblocks = end > begin ? (end - begin + kDecodeBlock - 1) / kDecodeBlock : 0;

    // ---- the small loads first (scales of the split, this wave's query chunk), then
    // the first K/V block: waits on the memory counter are in order, so the set-up
    // below never waits for the block
    // (a fixed count of loads, no branches: the counter waits below stay exact;
    // indices past the split repeat its last token, a cache hit)
    const uint32_t last = (end > begin ? end : length) - 1;
    float ksv[kMaxSplitTokens / 256], vsv[kMaxSplitTokens / 256];
#pragma unroll
    for (int it = 0; it < kMaxSplitTokens / 256; it++) {
        const size_t at = (size_t)min(begin + tid + 256 * it, last) * 2 + g;
        ksv[it] = p.ks[at];
        vsv[it] = p.vs[at];
    }
    // query chunk c = wave: lane (n, qq) takes dims 64c + 16qq + [0, 16) of head n % 8
    float4 x[4];
    {
        const float *qh = p.q + ((size_t)row * 16 + g * 8 + head) * 256 + 64 * wave + 16 * qq;
#pragma unroll
        for (int f = 0; f < 4; f++) x[f] = *reinterpret_cast<const float4 *>(qh + 4 * f);
    }
    // unconditional (a wave without blocks re-reads the first one, a cache hit): the
    // counter waits stay exact
    DecodeBlock cur, nxt;
    load_block(cur, p, g, begin + ((uint32_t)wave < nblocks ? wave : 0) * kDecodeBlock, length, lane, n, qq);

    // ---- scales of the split (this group) into LDS, vs_ref = their maximum; the
    // per-head maxima of the query chunks
    float vmax = 0.0f;
#pragma unroll
    for (int it = 0; it < kMaxSplitTokens / 256; it++) {
        const uint32_t e = tid + 256 * it;   // < kMaxSplitTokens; entries past the split are never read
        // masked by a multiply, not a select: every load above stays unconditional
        // (the clamped indices never reach a poisoned, non-finite tail scale)
        const float inside = begin + e < end ? 1.0f : 0.0f;
        kscale[e] = ksv[it] * (kLog2e / 16.0f) * inside;
        vscale[e] = vsv[it] * inside;
        vmax = fmaxf(vmax, vsv[it] * inside);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) vmax = fmaxf(vmax, __shfl_xor(vmax, o, 64));
    if (lane == 0) red[wave] = vmax;
    float amax = 0.0f;
#pragma unroll
    for (int f = 0; f < 4; f++) amax = fmaxf(amax, fmaxf(fmaxf(fabsf(x[f].x), fabsf(x[f].y)), fmaxf(fabsf(x[f].z), fabsf(x[f].w))));
    amax = fmaxf(amax, __shfl_xor(amax, 16, 64));
    amax = fmaxf(amax, __shfl_xor(amax, 32, 64));
    if (lane < 8) qmax[wave][lane] = amax;
    __syncthreads();
    const float vs_ref = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const float vs_inv = vs_ref > 0.0f ? 1.0f / vs_ref : 0.0f;
    // ---- INT8 query operand of chunk c = wave: part n / 8 of q ~= s_q (q1 + q2 / 254)
    const float qabs = fmaxf(fmaxf(qmax[0][head], qmax[1][head]), fmaxf(qmax[2][head], qmax[3][head]));
    const float qsc = qabs * (1.0f / 127.0f);   // s_q of the lane's head
    {
        const float inv = qabs > 0.0f ? 127.0f / qabs : 0.0f;
        auto part = [&](float v) {
            const float z = v * inv, q1 = rintf(z);
            const float q = lo_col ? rintf((z - q1) * 254.0f) : q1;
            return (uint32_t)(uint8_t)(int8_t)(int)fminf(fmaxf(q, -127.0f), 127.0f);
        };
        uint32_t w[4];
#pragma unroll
        for (int f = 0; f < 4; f++) w[f] = part(x[f].x) | (part(x[f].y) << 8) | (part(x[f].z) << 16) | (part(x[f].w) << 24);
        qlds[wave][lane] = v4i{(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
    }
    __syncthreads();
    v4i qi[4];
#pragma unroll
    for (int c = 0; c < 4; c++) qi[c] = qlds[c][lane];

    floatx4 o[16];
#pragma unroll
    for (int i = 0; i < 16; i++) o[i] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    float m = -INFINITY, l = 0.0f;

    for (uint32_t b = wave; b < nblocks; b += kDecodeWaves) {
        const uint32_t t0 = begin + b * kDecodeBlock;
        const bool more = b + kDecodeWaves < nblocks;            // wave-uniform
        // the last block re-reads itself (a cache hit) rather than branching
        load_block(nxt, p, g, more ? t0 + kDecodeWaves * kDecodeBlock : t0, length, lane, n, qq);
        v4i s[2];
#pragma unroll
        for (int a = 0; a < 2; a++) {
            v4i acc = {0, 0, 0, 0};
#pragma unroll
            for (int j = 0; j < 4; j++)
                acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(v4i, cur.k[a][j]), qi[j], acc, 0, 0, 0);
            s[a] = acc;
        }
        // C layout: lane (n, qq) holds rows 4*qq + r -> token t0 + 8*qq + 4*a + r; the
        // partner column n ^ 8 holds the other part of the same head.
        const int local0 = (int)(t0 - begin) + 8 * qq;          // token offset inside the split
        float sc[8];
        float top = -INFINITY;
#pragma unroll
        for (int a = 0; a < 2; a++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int mine = s[a][r], other = __shfl_xor(mine, 8, 64);
                const float full = ((float)(lo_col ? other : mine) + (float)(lo_col ? mine : other) * (1.0f / 254.0f)) * qsc;
                const uint32_t t = t0 + 8 * qq + 4 * a + r;
                const float value = t < end ? full * kscale[local0 + 4 * a + r] : -INFINITY;
                sc[a * 4 + r] = value;
                top = fmaxf(top, value);
            }
        top = fmaxf(top, __shfl_xor(top, 16, 64));
        top = fmaxf(top, __shfl_xor(top, 32, 64));
        const float next = fmaxf(m, top);
        const float decay = __builtin_amdgcn_exp2f(m - next);
        float total = 0.0f;
        uint32_t pw[4];
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
            _Float16 hv[2];
#pragma unroll
            for (int u = 0; u < 2; u++) {
                const float prob = __builtin_amdgcn_exp2f(sc[e + u] - next);   // 0 for masked tokens
                total += prob;
                const float scaled = prob * (vscale[local0 + e + u] * vs_inv);
                const _Float16 hi = (_Float16)scaled;
                hv[u] = lo_col ? (_Float16)(scaled - (float)hi) : hi;
            }
            const half2v ph = {hv[0], hv[1]};
            pw[e / 2] = __builtin_bit_cast(uint32_t, ph);
        }
        total += __shfl_xor(total, 16, 64);
        total += __shfl_xor(total, 32, 64);
        l = l * decay + total;
        m = next;
        if (decay != 1.0f) {
#pragma unroll
            for (int i = 0; i < 16; i++) o[i] *= decay;
        }
        const half8 pop = __builtin_bit_cast(half8, make_uint4(pw[0], pw[1], pw[2], pw[3]));
#pragma unroll
        for (int dt = 0; dt < 16; dt++)
            o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(i8x8_to_half8(cur.v[dt].x, cur.v[dt].y), pop, o[dt], 0, 0, 0);
        // the copy waits for the prefetched block: keep it after this block's MFMAs
        __builtin_amdgcn_sched_barrier(0);
        cur = nxt;
    }

    // ---- merge the four waves: O^T[d][n] with d = 16*dt + 4*qq + r; heads sum hi + lo columns;
    // statistics are in base 2, O in units of vs_ref.
    if (n < 8) {
#pragma unroll
        for (int dt = 0; dt < 16; dt++)
            *reinterpret_cast<floatx4 *>(&merge_o[wave][head][16 * dt + 4 * qq]) = o[dt];
        if (qq == 0) {
            merge_m[wave][head] = m;
            merge_l[wave][head] = l;
        }
    }
    __syncthreads();
    if (n >= 8) {
#pragma unroll
        for (int dt = 0; dt < 16; dt++) *reinterpret_cast<floatx4 *>(&merge_o[wave][head][16 * dt + 4 * qq]) += o[dt];
    }
    __syncthreads();
    // thread -> (head h, 8 dims); combine waves with their maxima
    const int h = threadIdx.x >> 5, d0 = (threadIdx.x & 31) * 8;
    float mw = -INFINITY;
    for (int w = 0; w < kDecodeWaves; w++) mw = fmaxf(mw, merge_m[w][h]);
    float lw = 0.0f, f[kDecodeWaves];
    for (int w = 0; w < kDecodeWaves; w++) {
        f[w] = merge_m[w][h] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(merge_m[w][h] - mw);
        lw += merge_l[w][h] * f[w];
    }
    float acc[8];
    for (int e = 0; e < 8; e++) {
        float sum = 0.0f;
        for (int w = 0; w < kDecodeWaves; w++) sum += merge_o[w][h][d0 + e] * f[w];
        acc[e] = sum * vs_ref;
    }
    if (p.splits == 1) {
        const size_t at = ((size_t)row * 16 + g * 8 + h) * 256 + d0;
        for (int e = 0; e < 8; e++) p.y[at + e] = acc[e] / lw * sigmoidf(p.gate[at + e]);
        return;
    }
    float *part = p.partial + (((size_t)row * 2 + g) * p.splits + split) * kPartialFloats;
    *reinterpret_cast<float4 *>(part + h * 256 + d0) = make_float4(acc[0], acc[1], acc[2], acc[3]);
    *reinterpret_cast<float4 *>(part + h * 256 + d0 + 4) = make_float4(acc[4], acc[5], acc[6], acc[7]);
    if ((threadIdx.x & 31) == 0) {
        part[2048 + h] = mw;
        part[2056 + h] = lw;
    }
}

// Merges the splits of one (row, head) for 64 dimensions (grid: 4 dimension
// chunks x 16 heads x rows). Two memory round trips: thread s first loads m_s
// and l_s of every split at once (the block maximum, the weights
// exp2(m_s - max) into LDS and the weighted sum of l), then 4 groups of 64 lanes
// stream the float4 partials of every 4th split and the groups are added in LDS.
__global__ __launch_bounds__(256) void decode_combine_kernel(const float *__restrict__ partial, const float *__restrict__ gate,
                                                             float *__restrict__ y, uint32_t splits) {
    __shared__ float weight[kMaxDecodeSplits];
    __shared__ float red[4], lred[4];
    __shared__ float4 sums[4][16];
    const uint32_t row = blockIdx.z, hq = blockIdx.y, g = hq / 8, h = hq % 8;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const float *base = partial + ((size_t)row * 2 + g) * splits * kPartialFloats;
    constexpr int kPer = kMaxDecodeSplits / 256;
    float ms[kPer], ls[kPer];
#pragma unroll
    for (int i = 0; i < kPer; i++) {
        const uint32_t sidx = min((uint32_t)(tid + 256 * i), splits - 1);
        ms[i] = tid + 256 * i < (int)splits ? base[(size_t)sidx * kPartialFloats + 2048 + h] : -INFINITY;
        ls[i] = base[(size_t)sidx * kPartialFloats + 2056 + h];
    }
    float mmax = -INFINITY;
#pragma unroll
    for (int i = 0; i < kPer; i++) mmax = fmaxf(mmax, ms[i]);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) mmax = fmaxf(mmax, __shfl_xor(mmax, o, 64));
    if (lane == 0) red[wave] = mmax;
    __syncthreads();
    mmax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    float lsum = 0.0f;
#pragma unroll
    for (int i = 0; i < kPer; i++) {
        if (tid + 256 * i >= (int)splits) continue;
        const float w = ms[i] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(ms[i] - mmax);
        weight[tid + 256 * i] = w;
        lsum += ls[i] * w;
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) lsum += __shfl_xor(lsum, o, 64);
    if (lane == 0) lred[wave] = lsum;
    __syncthreads();
    lsum = (lred[0] + lred[1]) + (lred[2] + lred[3]);
    // group `wave` takes splits wave, wave + 4, ...; lane: 4 dims of the 64-dim chunk
    const uint32_t d = blockIdx.x * 64 + 4 * (lane & 15);
    const int sub = lane >> 4;   // 4 sub-lanes per dim quad: splits wave + 4 (4j + sub)
    const float *col = base + (size_t)h * 256 + d;
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (uint32_t s0 = wave + 4 * sub; s0 < splits; s0 += 64) {
        float4 v[4];
        float w[4];
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const uint32_t sidx = s0 + 16 * u;
            const bool in = sidx < splits;
            v[u] = *reinterpret_cast<const float4 *>(col + (size_t)min(sidx, splits - 1) * kPartialFloats);
            w[u] = in ? weight[sidx] : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < 4; u++) {
            acc.x += v[u].x * w[u];
            acc.y += v[u].y * w[u];
            acc.z += v[u].z * w[u];
            acc.w += v[u].w * w[u];
        }
    }
    // the 16 (wave, sub) partial sums of each dim quad
#pragma unroll
    for (int o = 16; o < 64; o <<= 1) {
        acc.x += __shfl_xor(acc.x, o, 64);
        acc.y += __shfl_xor(acc.y, o, 64);
        acc.z += __shfl_xor(acc.z, o, 64);
        acc.w += __shfl_xor(acc.w, o, 64);
    }
    if (sub == 0) sums[wave][lane] = acc;
    __syncthreads();
    if (tid < 16) {
        float4 t = sums[0][tid];
#pragma unroll
        for (int w = 1; w < 4; w++) {
            t.x += sums[w][tid].x;
            t.y += sums[w][tid].y;
            t.z += sums[w][tid].z;
            t.w += sums[w][tid].w;
        }
        const size_t at = ((size_t)row * 16 + hq) * 256 + blockIdx.x * 64 + 4 * tid;
        const float inv = 1.0f / lsum;
        y[at + 0] = t.x * inv * sigmoidf(gate[at + 0]);   // y and gate need only 4-byte alignment
        y[at + 1] = t.y * inv * sigmoidf(gate[at + 1]);
        y[at + 2] = t.z * inv * sigmoidf(gate[at + 2]);
        y[at + 3] = t.w * inv * sigmoidf(gate[at + 3]);
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
    dim3 grid((uint32_t)((K + 63) / 64), (uint32_t)(rows * 2));
    scores_int8_kernel<<<grid, 64, 0, context_stream(c)>>>((const float *)b[0].ptr, (const int8_t *)b[1].ptr,
                                                           (float *)b[2].ptr, (const float *)b[3].ptr, (uint32_t)rows,
                                                           (uint32_t)K, p.pos);
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
    softmax_kernel<<<(uint32_t)groups, 256, 0, context_stream(c)>>>((float *)b[0].ptr, (uint32_t)K, p.pos);
    return nullptr;
}

const char *launch_values_int8(Context &c, const View *b, int count, const boot_kernel_args &p, const uint32_t *) {
    // bindings: scores, v INT8 pages, gate, y, vs (QwenEngine.cs:165, Prefill.cs:283)
    BOOT_REQUIRE(count >= 5, "batch_attention_values_int8 needs 5 bindings: scores, v, gate, y, vs");
    const uint64_t rows = p.m, K = p.k;
    if (rows == 0) return nullptr;
    const uint64_t length = (uint64_t)p.pos + rows;
    BOOT_REQUIRE(length <= K, "causal end pos+rows exceeds the score row stride K");
    BOOT_REQUIRE(b[0].bytes >= rows * 16 * K * 4, "scores buffer smaller than rows*16*K floats");
    BOOT_REQUIRE(b[1].bytes >= value_bytes(length), "V cache smaller than whole pages of the attended length");
    BOOT_REQUIRE(b[2].bytes >= rows * 16384 && b[3].bytes >= rows * 16384, "gate/output smaller than rows*4096 floats");
    BOOT_REQUIRE(b[4].bytes >= length * 8, "V scale buffer smaller than the attended length");
    BOOT_REQUIRE(aligned(b[1].ptr, 16), "V cache binding must be 16-byte aligned");
    const uint64_t threads = rows * 4096;
    values_int8_kernel<<<(uint32_t)((threads + 255) / 256), 256, 0, context_stream(c)>>>(
        (const float *)b[0].ptr, (const int8_t *)b[1].ptr, (const float *)b[2].ptr, (float *)b[3].ptr,
        (const float *)b[4].ptr, (uint32_t)rows, (uint32_t)K, p.pos);
    return nullptr;
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
    // Split length in 32-token blocks, chosen so that the grid (splits x 2 groups x
    // rows, two work-groups per CU) fits the CUs in one round: a second, nearly empty
    // round would double the time. At most kMaxSplitTokens per split.
    const uint64_t total_blocks = (length + kDecodeBlock - 1) / kDecodeBlock;
    const uint64_t slots = std::max<uint64_t>(1, 2ull * (uint64_t)std::max(1, context_cus(c)) / (2 * rows));
    uint64_t split_blocks = (total_blocks + slots - 1) / slots;
    split_blocks = std::max<uint64_t>(split_blocks, (uint64_t)kDecodeWaves);             // one block per wave at least
    split_blocks = std::min<uint64_t>(split_blocks, (uint64_t)(kMaxSplitTokens / kDecodeBlock));
    const uint64_t splits = (total_blocks + split_blocks - 1) / split_blocks;
    BOOT_REQUIRE(splits <= kMaxDecodeSplits, "too many decode splits");
    DecodeParams d;
    d.q = (const float *)b[0].ptr;
    d.k = (const int8_t *)b[1].ptr;
    d.v = (const int8_t *)b[2].ptr;
    d.gate = (const float *)b[3].ptr;
    d.y = (float *)b[4].ptr;
    d.ks = (const float *)b[5].ptr;
    d.vs = (const float *)b[6].ptr;
    d.rows = (uint32_t)rows;
    d.pos = p.pos;
    d.splits = (uint32_t)splits;
    d.split_blocks = (uint32_t)split_blocks;
    d.partial = nullptr;
    if (splits > 1) {
        d.partial = (float *)context_workspace(c, rows * 2 * splits * kPartialFloats * sizeof(float));
        BOOT_REQUIRE(d.partial, "cannot allocate decode split workspace");
    }
    decode_int8_kernel<<<dim3((uint32_t)splits, 2, (uint32_t)rows), 256, 0, context_stream(c)>>>(d);
    if (splits > 1) {
        context_split(c, "attention_decode_int8.combine");
        decode_combine_kernel<<<dim3(4, 16, (uint32_t)rows), 256, 0, context_stream(c)>>>(d.partial, d.gate, d.y,
                                                                                        (uint32_t)splits);
    }
    return nullptr;
}

}  // namespace boot
