// INT8 KV append (quantize + store), partial RoPE, grouped FP16 query packing
// and the zero fill. gfx950, wave64.
//
// Reference semantics:
//   store_kv_int8            kernels.metal:129-141
//   int8_value_index         kernels.metal:126-128
//   rotated (partial RoPE)   kernels.metal:122-125
//   batch_rope_int8          kernels.metal:142-146
//   attention_query_grouped_half  kernels.metal:1276-1281
//
// Bit-exactness of codes and scales: amax is an exact max; the scale is the
// correctly rounded fp32 quotient amax/127 and codes are rint(x * (127/amax))
// with one correctly rounded quotient and one fp32 multiply, clamped to
// +-127. The library is built without fast-math, with correctly rounded fp32
// division, so these are the IEEE operations the reference specifies.
#include "common.h"
#include "kvmath.h"
#include "mfma.h"

namespace boot {
namespace {

// A read-once float4 (non-temporal load: it need not displace anything in L2)
__device__ __attribute__((always_inline)) inline float4 load_once4(const float *at) {
    typedef float f32x4_t __attribute__((ext_vector_type(4)));
    return __builtin_bit_cast(float4, __builtin_nontemporal_load(reinterpret_cast<const f32x4_t *>(at)));
}

constexpr int kTile = 16;               // tokens per store work-group (page-aligned tiles): 4 per wave
constexpr int kBulkTile = 64;           // tile of large appends: whole 64-byte V page-row runs
constexpr uint64_t kBulkRows = 4096;    // appends of at least this many rows use kBulkTile
// Bytes per LDS row of the V transpose: the tile plus 4, an odd number of dwords, so the
// byte writes of a wave's 64 rows fall in 64 different banks.
template <int Tile>
constexpr int vt_stride() { return Tile + 4; }



// Quantizes and appends tokens [lo, hi) of one Tile-token tile for one KV head.
// K: one wave per token, float4 per lane, codes written token-major as char4.
// V: codes transposed in LDS, then written as page rows (Tile-byte runs for a full
// tile, byte stores at partial tile edges), kernels.metal:126-128. Short runs cost
// write bandwidth: 16-byte runs wrote 1.6x the bytes of a bulk append.
template <bool Rope, bool Norm = false, int Tile = kTile>
__device__ void store_tile(const float *__restrict__ k, const float *__restrict__ v,
                           int8_t *__restrict__ kc, int8_t *__restrict__ vc,
                           float *__restrict__ ks, float *__restrict__ vs,
                           uint32_t rows, uint32_t pos, uint32_t tile, uint32_t h,
                           uint8_t *vt, float ifreq, KNorm knorm = {nullptr, 0.0f}) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    constexpr int kVtStride = vt_stride<Tile>();
    const uint32_t tile0 = tile * Tile;
    const uint32_t lo = max(tile0, pos), hi = min(tile0 + Tile, pos + rows);
    // Each pass, wave w takes tokens w, w + 4, w + 8, ... of the tile, kPer of them, whose loads
    // are issued before any is quantized so that the requests are in flight together (bulk tiles:
    // 8 per pass, 117.6-118.7 against 120.4-120.8 us for 131072 tokens with 4; 16: 134 us).
    constexpr int kPer = Tile >= 64 ? 8 : 4;
    for (uint32_t tb = wave; tb < Tile; tb += 4 * kPer) {
        float4 kx[kPer];
        float vx[kPer][4];
#pragma unroll
        for (int u = 0; u < kPer; u++) {
            const uint32_t t = min(max(tile0 + tb + 4 * u, lo), hi - 1);   // in-range row for the load
            const uint32_t row = t - pos;
            const float *kr = k + ((size_t)row * 2 + h) * 256;
            const float *vr = v + ((size_t)row * 2 + h) * 256;
            kx[u] = load_once4(kr + 4 * lane);
#pragma unroll
            for (int i = 0; i < 4; i++) vx[u][i] = __builtin_nontemporal_load(vr + lane + 64 * i);
        }
        // The pass's token chains (norm, rotation, two wave maxima: cross-lane steps with memory-like
        // latency) are computed together, with no branch between them, so that they overlap; only
        // the stores are skipped for tokens outside [lo, hi) (their loads read an in-range row).
        float4 kq[kPer];
        float kam[kPer], vam[kPer];
#pragma unroll
        for (int u = 0; u < kPer; u++) {
            float4 kv = kx[u];
            if (Norm) kv = rms_norm4(kv, knorm.eps, knorm.w, lane, 1.0f);
            if (Rope) kv = rope4(kv, lane, rope_angles(tile0 + tb + 4 * u, lane, ifreq));
            kam[u] = wave_max(fmaxf(fmaxf(fabsf(kv.x), fabsf(kv.y)), fmaxf(fabsf(kv.z), fabsf(kv.w))));
            vam[u] = wave_max(fmaxf(fmaxf(fabsf(vx[u][0]), fabsf(vx[u][1])), fmaxf(fabsf(vx[u][2]), fabsf(vx[u][3]))));
            kq[u] = kv;
        }
#pragma unroll
        for (int u = 0; u < kPer; u++) {
            const uint32_t tl = tb + 4 * u, t = tile0 + tl;
            if (t < lo || t >= hi) continue;  // wave-uniform
            const float4 kv = kq[u];
            const float ka = kam[u], va = vam[u];
            const uint64_t vector = (uint64_t)t * 2 + h;
            if (lane == 0) {
                ks[vector] = ka / 127.0f;
                vs[vector] = va / 127.0f;
            }
            const float kr127 = 127.0f / ka, vr127 = 127.0f / va;
            *reinterpret_cast<uint32_t *>(kc + vector * 256 + 4 * lane) =
                pack4(quant_code(kv.x, ka, kr127), quant_code(kv.y, ka, kr127),
                      quant_code(kv.z, ka, kr127), quant_code(kv.w, ka, kr127));
#pragma unroll
            for (int i = 0; i < 4; i++)
                vt[(lane + 64 * i) * kVtStride + tl] = (uint8_t)(int8_t)(int)quant_code(vx[u][i], va, vr127);
        }
    }
    __syncthreads();
    const uint64_t base = ((uint64_t)(tile0 >> 8) * 2 + h) * kPageBytes + (tile0 & 255);
    if (lo == tile0 && hi == tile0 + Tile) {
        // thread d writes the tile's Tile bytes of page row d
        const int d = threadIdx.x;
        const uint32_t *src = reinterpret_cast<const uint32_t *>(vt + d * kVtStride);
#pragma unroll
        for (int q = 0; q < Tile / 16; q++)
            *reinterpret_cast<uint4 *>(vc + base + (uint64_t)d * 256 + 16 * q) =
                make_uint4(src[4 * q], src[4 * q + 1], src[4 * q + 2], src[4 * q + 3]);
    } else {
        // partial tile (chunk edges, single-token decode appends): only the valid bytes
        const uint32_t count = hi - lo, first = lo - tile0;
        for (uint32_t item = threadIdx.x; item < 256 * count; item += 256) {
            const uint32_t d = item / count, tl = first + item % count;
            vc[base + (uint64_t)d * 256 + tl] = vt[d * kVtStride + tl];
        }
    }
}

template <int Tile>
__global__ __launch_bounds__(256) void kv_store_int8_kernel(
    const float *__restrict__ k, const float *__restrict__ v, int8_t *__restrict__ kc,
    int8_t *__restrict__ vc, float *__restrict__ ks, float *__restrict__ vs, uint32_t rows,
    uint32_t pos, uint32_t first_tile) {
    __shared__ __attribute__((aligned(16))) uint8_t vt[256 * vt_stride<Tile>()];
    store_tile<false, false, Tile>(k, v, kc, vc, ks, vs, rows, pos, first_tile + blockIdx.x / 2, blockIdx.x & 1,
                                   vt, 0.0f);
}

// batch_rope_int8 (kernels.metal:142-146): the first blocks rotate K and append
// the K/V tiles; the last qblocks rotate the 16 query heads of every row into
// qr. One launch.
__global__ __launch_bounds__(256) void batch_rope_int8_kernel(
    const float *__restrict__ q, const float *__restrict__ k, const float *__restrict__ v,
    float *__restrict__ qr, int8_t *__restrict__ kc, int8_t *__restrict__ vc,
    float *__restrict__ ks, float *__restrict__ vs, uint32_t rows, uint32_t pos, RopeFreq freq,
    uint32_t qblocks, uint32_t first_tile) {
    __shared__ __attribute__((aligned(16))) uint8_t vt[256 * vt_stride<kTile>()];
    const float ifreq = lane_inv_freq(freq);
    const uint32_t kvblocks = gridDim.x - qblocks;   // K/V tiles first, as prepare_fused_int8_kernel
    if (blockIdx.x >= kvblocks) {
        // one work-group per row, wave w rotating heads 4w..4w+3 (loads issued together)
        const int lane = threadIdx.x & 63, h0 = 4 * (threadIdx.x >> 6);
        const uint32_t row = blockIdx.x - kvblocks;
        const Rope4 r = rope_angles(pos + row, lane, ifreq);
        const float *src = q + (size_t)row * 4096 + h0 * 256 + 4 * lane;
        float *dst = qr + (size_t)row * 4096 + h0 * 256 + 4 * lane;
        float4 x[4];
#pragma unroll
        for (int h = 0; h < 4; h++) x[h] = *reinterpret_cast<const float4 *>(src + h * 256);
#pragma unroll
        for (int h = 0; h < 4; h++) *reinterpret_cast<float4 *>(dst + h * 256) = rope4(x[h], lane, r);
        return;
    }
    const uint32_t b = blockIdx.x;
    store_tile<true>(k, v, kc, vc, ks, vs, rows, pos, first_tile + b / 2, b & 1, vt, ifreq);
}

// attention_prepare_fused_int8 (kernels.metal:1902-1914): per row, the 16
// query heads (RMS norm with q_norm, RoPE, FP16 into the grouped layout, gate
// split) and the 2 KV heads (RMS norm with k_norm, RoPE, INT8 append). One wave
// per row rotates its 16 query heads with one set of angles; K/V use the
// page-tiled store. q holds [rows][16][q 256 | gate 256] (kernels.metal:1904).
// Query half of the fused preparations (kernels.metal:1896-1900 / 1907-1911): work-group `row`,
// wave w takes heads 4w..4w+3 with all their loads issued together; each head is RMS-normalized
// with (w + 1), rotated, written as grouped FP16 [(h/8*rows+row)*8+h%8][256], and its gate half
// copied out. The per-head arithmetic is rmsnorm's and batch_rope_int8's, so the fused and the
// unfused chains give the same bits.
__device__ __attribute__((always_inline)) inline void prepare_query_heads(
    const float *__restrict__ qkv, const uint16_t *__restrict__ qw, _Float16 *__restrict__ packed,
    float *__restrict__ gate, uint32_t rows, uint32_t row, uint32_t pos, float eps, float ifreq) {
    typedef _Float16 half4 __attribute__((ext_vector_type(4)));
    const int lane = threadIdx.x & 63, h0 = 4 * (threadIdx.x >> 6);
    const Rope4 r = rope_angles(pos + row, lane, ifreq);
    const float *src = qkv + (size_t)row * 8192 + h0 * 512 + 4 * lane;
    float4 x[4], gv[4];
#pragma unroll
    for (int h = 0; h < 4; h++) {
        x[h] = *reinterpret_cast<const float4 *>(src + h * 512);
        gv[h] = *reinterpret_cast<const float4 *>(src + h * 512 + 256);
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int h = h0 + i;
        const float4 z = rope4(rms_norm4(x[i], eps, qw, lane, 1.0f), lane, r);
        const half4 hz = {(_Float16)z.x, (_Float16)z.y, (_Float16)z.z, (_Float16)z.w};
        *reinterpret_cast<half4 *>(packed + (((size_t)(h / 8) * rows + row) * 8 + h % 8) * 256 + 4 * lane) = hz;
        *reinterpret_cast<float4 *>(gate + ((size_t)row * 16 + h) * 256 + 4 * lane) = gv[i];
    }
}

__global__ __launch_bounds__(256) void prepare_fused_int8_kernel(
    const float *__restrict__ qkv, const float *__restrict__ k, const float *__restrict__ v,
    const uint16_t *__restrict__ qw, const uint16_t *__restrict__ kw, _Float16 *__restrict__ packed,
    float *__restrict__ gate, int8_t *__restrict__ kc, int8_t *__restrict__ vc, float *__restrict__ ks,
    float *__restrict__ vs, uint32_t rows, uint32_t pos, RopeFreq freq, float eps, uint32_t qblocks,
    uint32_t first_tile) {
    __shared__ __attribute__((aligned(16))) uint8_t vt[256 * vt_stride<kTile>()];
    const float ifreq = lane_inv_freq(freq);
    // The K/V tiles come first in the grid: their chain (loads, norm, RoPE, two wave maxima, the
    // V transpose) is the launch's longest, and dispatched behind the query rows they ran last.
    const uint32_t kvblocks = gridDim.x - qblocks;
    if (blockIdx.x >= kvblocks) {
        prepare_query_heads(qkv, qw, packed, gate, rows, blockIdx.x - kvblocks, pos, eps, ifreq);
        return;
    }
    const uint32_t b = blockIdx.x;
    store_tile<true, true>(k, v, kc, vc, ks, vs, rows, pos, first_tile + b / 2, b & 1, vt, ifreq, KNorm{kw, eps});
}

// batch_rope with FP16 KV storage (flags bit 256; kernels.metal:16-21, 322-324):
// rotated Q in FP32, rotated K and V rounded to FP16 into the token-major
// [cap][2][256] control cache. One wave per row; angles computed once per row.
// FP16-KV fused preparation (attention_prepare_fused, kernels.metal:1889-1901): per token row,
// the 16 query heads RMS-normalized with (w + 1), rotated, packed as grouped FP16 with the gate
// split out (as prepare_fused_int8_kernel), and the 2 K heads normalized, rotated and stored with
// V as FP16, token-major [pos + row][2][256] (kernels.metal:16-21). One wave per row.
__global__ __launch_bounds__(256) void prepare_fused_half_kernel(
    const float *__restrict__ qkv, const float *__restrict__ k, const float *__restrict__ v,
    const uint16_t *__restrict__ qw, const uint16_t *__restrict__ kw, _Float16 *__restrict__ packed,
    float *__restrict__ gate, _Float16 *__restrict__ kc, _Float16 *__restrict__ vc, uint32_t rows, uint32_t pos,
    RopeFreq freq, float eps) {
    const float ifreq = lane_inv_freq(freq);
    if (blockIdx.x < rows) {
        prepare_query_heads(qkv, qw, packed, gate, rows, blockIdx.x, pos, eps, ifreq);
        return;
    }
    // K/V: one wave per row
    const int lane = threadIdx.x & 63;
    const uint32_t row = (blockIdx.x - rows) * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;                                         // wave-uniform
    const Rope4 r = rope_angles(pos + row, lane, ifreq);
    typedef _Float16 half4 __attribute__((ext_vector_type(4)));
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const size_t src = (size_t)row * 512 + h * 256 + 4 * lane, dst = ((size_t)(pos + row) * 2 + h) * 256 + 4 * lane;
        const float4 kz = rope4(rms_norm4(*reinterpret_cast<const float4 *>(k + src), eps, kw, lane, 1.0f), lane, r);
        const float4 vz = *reinterpret_cast<const float4 *>(v + src);
        const half4 kh = {(_Float16)kz.x, (_Float16)kz.y, (_Float16)kz.z, (_Float16)kz.w};
        const half4 vh = {(_Float16)vz.x, (_Float16)vz.y, (_Float16)vz.z, (_Float16)vz.w};
        *reinterpret_cast<half4 *>(kc + dst) = kh;
        *reinterpret_cast<half4 *>(vc + dst) = vh;
    }
}

__global__ __launch_bounds__(256) void batch_rope_half_kernel(const float *__restrict__ q, const float *__restrict__ k,
                                                              const float *__restrict__ v, float *__restrict__ qr,
                                                              _Float16 *__restrict__ kc, _Float16 *__restrict__ vc,
                                                              uint32_t rows, uint32_t pos, RopeFreq freq) {
    const float ifreq = lane_inv_freq(freq);
    const int lane = threadIdx.x & 63;
    const uint32_t row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;                                         // wave-uniform
    const Rope4 r = rope_angles(pos + row, lane, ifreq);
    typedef _Float16 half4 __attribute__((ext_vector_type(4)));
#pragma unroll 4
    for (int h = 0; h < 16; h++) {
        const size_t at = (size_t)row * 4096 + h * 256 + 4 * lane;
        *reinterpret_cast<float4 *>(qr + at) = rope4(*reinterpret_cast<const float4 *>(q + at), lane, r);
    }
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const size_t src = (size_t)row * 512 + h * 256 + 4 * lane, dst = ((size_t)(pos + row) * 2 + h) * 256 + 4 * lane;
        const float4 kz = rope4(*reinterpret_cast<const float4 *>(k + src), lane, r);
        const float4 vz = *reinterpret_cast<const float4 *>(v + src);
        const half4 kh = {(_Float16)kz.x, (_Float16)kz.y, (_Float16)kz.z, (_Float16)kz.w};
        const half4 vh = {(_Float16)vz.x, (_Float16)vz.y, (_Float16)vz.z, (_Float16)vz.w};
        *reinterpret_cast<half4 *>(kc + dst) = kh;
        *reinterpret_cast<half4 *>(vc + dst) = vh;
    }
}

// rmsnorm (kernels.metal:51-57) for 256-wide groups, one wave per group:
// y = x * rsqrt-mean-square * (w + offset) [* silu(gate) with flag 2].
__global__ __launch_bounds__(256) void rmsnorm256_kernel(const float *__restrict__ x, const uint16_t *__restrict__ w,
                                                         float *__restrict__ y, const float *__restrict__ gate,
                                                         uint32_t groups, float eps, uint32_t flags) {
    const int lane = threadIdx.x & 63;
    const uint32_t group = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (group >= groups) return;
    const size_t at = (size_t)group * 256 + 4 * lane;
    float4 z = rms_norm4(*reinterpret_cast<const float4 *>(x + at), eps, w, lane, (flags & 1) ? 1.0f : 0.0f);
    if (flags & 2) {
        const float4 gv = *reinterpret_cast<const float4 *>(gate + at);
        z.x *= gv.x / (1.0f + expf(-gv.x));
        z.y *= gv.y / (1.0f + expf(-gv.y));
        z.z *= gv.z / (1.0f + expf(-gv.z));
        z.w *= gv.w / (1.0f + expf(-gv.w));
    }
    *reinterpret_cast<float4 *>(y + at) = z;
}

// batch_split_q (kernels.metal:321): [rows][16][q | gate] -> q [rows][16][256], gate [rows][16][256].
__global__ __launch_bounds__(256) void batch_split_q_kernel(const float *__restrict__ x, float *__restrict__ q,
                                                            float *__restrict__ gate, uint32_t rows) {
    const uint64_t i = ((uint64_t)blockIdx.x * 256 + threadIdx.x) * 4;
    if (i >= (uint64_t)rows * 4096) return;
    const uint64_t token = i / 4096, h = (i % 4096) / 256, d = i % 256;
    const float *src = x + token * 8192 + h * 512 + d;
    *reinterpret_cast<float4 *>(q + i) = *reinterpret_cast<const float4 *>(src);
    *reinterpret_cast<float4 *>(gate + i) = *reinterpret_cast<const float4 *>(src + 256);
}

__global__ __launch_bounds__(256) void query_grouped_half_kernel(const float *__restrict__ x,
                                                                 _Float16 *__restrict__ y,
                                                                 uint32_t rows, uint32_t group_log2) {
    // kernels.metal:1276-1281: y[(h / A) * M + row][h % A] = half(x[row][h]), eight values per
    // thread, read in source order; A is a power of two (it divides 16)
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i >= rows * 512) return;
    const uint32_t vec = i >> 5, d0 = (i & 31) * 8;              // vec = row * 16 + h
    const uint32_t row = vec >> 4, h = vec & 15;
    const uint32_t gmask = (1u << group_log2) - 1;
    const uint32_t dst = (((h >> group_log2) * rows + row) << group_log2) + (h & gmask);
    const float4 a = *reinterpret_cast<const float4 *>(x + (size_t)vec * 256 + d0);
    const float4 b = *reinterpret_cast<const float4 *>(x + (size_t)vec * 256 + d0 + 4);
    const half8 o = {(_Float16)a.x, (_Float16)a.y, (_Float16)a.z, (_Float16)a.w,
                     (_Float16)b.x, (_Float16)b.y, (_Float16)b.z, (_Float16)b.w};   // RNE
    *reinterpret_cast<half8 *>(y + (size_t)dst * 256 + d0) = o;
}

__global__ __launch_bounds__(256) void fill_zero_kernel(uint4 *__restrict__ p, uint64_t n16,
                                                        uint8_t *__restrict__ tail, uint32_t ntail) {
    const uint64_t stride = (uint64_t)gridDim.x * 256;
    for (uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x; i < n16; i += stride)
        p[i] = make_uint4(0, 0, 0, 0);
    if (blockIdx.x == 0 && threadIdx.x < ntail) tail[threadIdx.x] = 0;
}

inline bool aligned(const void *p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

const char *check_cache(const View *b, int kc, int vc, int ks, int vs, uint64_t end) {
    // end = one past the last token written
    if (end == 0) return nullptr;
    BOOT_REQUIRE(b[kc].bytes >= end * 512, "K cache buffer too small for position+rows");
    BOOT_REQUIRE(b[vc].bytes >= value_index((end - 1) * 2 + 1, 255) + 1,
                 "V cache buffer too small for position+rows (whole 256-token pages)");
    BOOT_REQUIRE(b[ks].bytes >= end * 8 && b[vs].bytes >= end * 8, "KV scale buffer too small");
    BOOT_REQUIRE(aligned(b[kc].ptr, 4) && aligned(b[vc].ptr, 16), "KV cache bindings must be 16-byte aligned");
    BOOT_REQUIRE(aligned(b[ks].ptr, 4) && aligned(b[vs].ptr, 4), "KV scale bindings must be 4-byte aligned");
    return nullptr;
}

}  // namespace

const char *launch_kv_store_int8(Context &c, const View *b, int count, const boot_kernel_args &p,
                                 const uint32_t *) {
    // bindings: k, v (FP32 [rows][2][256], post-RoPE), kc, vc, ks, vs
    BOOT_REQUIRE(count >= 6, "kv_store_int8 needs 6 bindings: k, v, kc, vc, ks, vs");
    const uint64_t rows = p.m, end = (uint64_t)p.pos + rows;
    if (rows == 0) return nullptr;
    BOOT_REQUIRE(b[0].bytes >= rows * 2048 && b[1].bytes >= rows * 2048, "K/V input smaller than rows*512 floats");
    BOOT_REQUIRE(aligned(b[0].ptr, 16) && aligned(b[1].ptr, 16), "K/V input bindings must be 16-byte aligned");
    if (const char *e = check_cache(b, 2, 3, 4, 5, end)) return e;
    const bool bulk = rows >= kBulkRows;
    const uint32_t tile = bulk ? kBulkTile : kTile;
    const uint32_t first = p.pos / tile, last = (uint32_t)((end - 1) / tile);
    const uint32_t blocks = (last - first + 1) * 2;
    if (bulk)
        launch_timed(c, "kv_store_int8_kernel", kv_store_int8_kernel<kBulkTile>, dim3(blocks), dim3(256),
                     (const float *)b[0].ptr, (const float *)b[1].ptr, (int8_t *)b[2].ptr, (int8_t *)b[3].ptr,
                     (float *)b[4].ptr, (float *)b[5].ptr, (uint32_t)rows, p.pos, first);
    else
        launch_timed(c, "kv_store_int8_kernel", kv_store_int8_kernel<kTile>, dim3(blocks), dim3(256),
                     (const float *)b[0].ptr, (const float *)b[1].ptr, (int8_t *)b[2].ptr, (int8_t *)b[3].ptr,
                     (float *)b[4].ptr, (float *)b[5].ptr, (uint32_t)rows, p.pos, first);
    return nullptr;
}

const char *launch_batch_rope_int8(Context &c, const View *b, int count, const boot_kernel_args &p,
                                   const uint32_t *) {
    // bindings: q, k, v, qr, kc, vc, ks, vs (kernels.metal:142, Prefill.cs:257, QwenEngine.cs:162)
    BOOT_REQUIRE(count >= 8, "batch_rope_int8 needs 8 bindings: q, k, v, qr, kc, vc, ks, vs");
    const uint64_t rows = p.m, end = (uint64_t)p.pos + rows;
    if (rows == 0) return nullptr;
    BOOT_REQUIRE(b[0].bytes >= rows * 16384 && b[3].bytes >= rows * 16384, "Q/rotated buffers smaller than rows*4096 floats");
    BOOT_REQUIRE(b[1].bytes >= rows * 2048 && b[2].bytes >= rows * 2048, "K/V input smaller than rows*512 floats");
    BOOT_REQUIRE(aligned(b[0].ptr, 16) && aligned(b[1].ptr, 16) && aligned(b[2].ptr, 16) && aligned(b[3].ptr, 16),
                 "Q/K/V bindings must be 16-byte aligned");
    if (const char *e = check_cache(b, 4, 5, 6, 7, end)) return e;
    const uint32_t qblocks = (uint32_t)rows;   // one work-group per row for the query heads
    const uint32_t first = p.pos / kTile, last = (uint32_t)((end - 1) / kTile);
    const uint32_t blocks = qblocks + (last - first + 1) * 2;
    launch_timed(c, "batch_rope_int8_kernel", batch_rope_int8_kernel, dim3(blocks), dim3(256), 
        (const float *)b[0].ptr, (const float *)b[1].ptr, (const float *)b[2].ptr, (float *)b[3].ptr,
        (int8_t *)b[4].ptr, (int8_t *)b[5].ptr, (float *)b[6].ptr, (float *)b[7].ptr, (uint32_t)rows,
        p.pos, rope_frequencies(p.theta), qblocks, first);
    return nullptr;
}

const char *launch_query_grouped_half(Context &c, const View *b, int count, const boot_kernel_args &p,
                                      const uint32_t *) {
    // bindings: x FP32 [rows][16][256], y FP16 grouped (DeviceAttention.cs:68)
    BOOT_REQUIRE(count >= 2, "attention_query_grouped_half needs 2 bindings: x, y");
    const uint64_t rows = p.m;
    if (rows == 0) return nullptr;
    BOOT_REQUIRE(p.a >= 1 && p.a <= 16 && 16 % p.a == 0, "group size A must divide 16");
    BOOT_REQUIRE(b[0].bytes >= rows * 16384 && b[1].bytes >= rows * 8192, "query buffers smaller than rows*4096 values");
    BOOT_REQUIRE(rows <= 262144, "rows exceed the 262144-token window");
    BOOT_REQUIRE(aligned(b[0].ptr, 16) && aligned(b[1].ptr, 16), "query bindings must be 16-byte aligned");
    const uint64_t threads = rows * 512;
    launch_timed(c, "query_grouped_half_kernel", query_grouped_half_kernel, dim3((uint32_t)((threads + 255) / 256)), dim3(256), 
        (const float *)b[0].ptr, (_Float16 *)b[1].ptr, (uint32_t)rows, (uint32_t)__builtin_ctz(p.a));
    return nullptr;
}

const char *launch_prepare_fused_int8(Context &c, const View *b, int count, const boot_kernel_args &p,
                                      const uint32_t *) {
    // bindings (Prefill.cs:250): qkv, k, v, q_norm w, k_norm w, packed Q, gate, kc, vc, ks, vs
    BOOT_REQUIRE(count >= 11, "attention_prepare_fused_int8 needs 11 bindings");
    const uint64_t rows = p.m, end = (uint64_t)p.pos + rows;
    if (rows == 0) return nullptr;
    BOOT_REQUIRE(b[0].bytes >= rows * 32768, "qkv input smaller than rows*8192 floats");
    BOOT_REQUIRE(b[1].bytes >= rows * 2048 && b[2].bytes >= rows * 2048, "K/V input smaller than rows*512 floats");
    BOOT_REQUIRE(b[3].bytes >= 512 && b[4].bytes >= 512, "norm weights smaller than 256 bf16");
    BOOT_REQUIRE(b[5].bytes >= rows * 8192, "packed query smaller than rows*4096 halves");
    BOOT_REQUIRE(b[6].bytes >= rows * 16384, "gate output smaller than rows*4096 floats");
    BOOT_REQUIRE(aligned(b[0].ptr, 16) && aligned(b[1].ptr, 16) && aligned(b[2].ptr, 16) && aligned(b[3].ptr, 8) &&
                     aligned(b[4].ptr, 8) && aligned(b[5].ptr, 8) && aligned(b[6].ptr, 16),
                 "bindings misaligned");
    if (const char *e = check_cache(b, 7, 8, 9, 10, end)) return e;
    const uint32_t qblocks = (uint32_t)rows;   // one work-group per row for the query heads
    const uint32_t first = p.pos / kTile, last = (uint32_t)((end - 1) / kTile);
    launch_timed(c, "prepare_fused_int8_kernel", prepare_fused_int8_kernel, dim3(qblocks + (last - first + 1) * 2), dim3(256), 
        (const float *)b[0].ptr, (const float *)b[1].ptr, (const float *)b[2].ptr, (const uint16_t *)b[3].ptr,
        (const uint16_t *)b[4].ptr, (_Float16 *)b[5].ptr, (float *)b[6].ptr, (int8_t *)b[7].ptr, (int8_t *)b[8].ptr,
        (float *)b[9].ptr, (float *)b[10].ptr, (uint32_t)rows, p.pos, rope_frequencies(p.theta), p.eps, qblocks, first);
    return nullptr;
}

const char *launch_prepare_fused_half(Context &c, const View *b, int count, const boot_kernel_args &p,
                                      const uint32_t *) {
    // bindings (Prefill.cs:252): qkv, k, v, q_norm w, k_norm w, packed Q, gate, kc, vc (FP16 [cap][2][256])
    BOOT_REQUIRE(count >= 9, "attention_prepare_fused needs 9 bindings");
    const uint64_t rows = p.m, end = (uint64_t)p.pos + rows;
    if (rows == 0) return nullptr;
    BOOT_REQUIRE(b[0].bytes >= rows * 32768, "qkv input smaller than rows*8192 floats");
    BOOT_REQUIRE(b[1].bytes >= rows * 2048 && b[2].bytes >= rows * 2048, "K/V input smaller than rows*512 floats");
    BOOT_REQUIRE(b[3].bytes >= 512 && b[4].bytes >= 512, "norm weights smaller than 256 bf16");
    BOOT_REQUIRE(b[5].bytes >= rows * 8192, "packed query smaller than rows*4096 halves");
    BOOT_REQUIRE(b[6].bytes >= rows * 16384, "gate output smaller than rows*4096 floats");
    BOOT_REQUIRE(b[7].bytes >= end * 1024 && b[8].bytes >= end * 1024, "FP16 KV cache smaller than position+rows");
    BOOT_REQUIRE(aligned(b[0].ptr, 16) && aligned(b[1].ptr, 16) && aligned(b[2].ptr, 16) && aligned(b[3].ptr, 8) &&
                     aligned(b[4].ptr, 8) && aligned(b[5].ptr, 8) && aligned(b[6].ptr, 16) && aligned(b[7].ptr, 8) &&
                     aligned(b[8].ptr, 8),
                 "bindings misaligned");
    launch_timed(c, "prepare_fused_half_kernel", prepare_fused_half_kernel, dim3((uint32_t)(rows + (rows + 3) / 4)), dim3(256),
        (const float *)b[0].ptr, (const float *)b[1].ptr, (const float *)b[2].ptr, (const uint16_t *)b[3].ptr,
        (const uint16_t *)b[4].ptr, (_Float16 *)b[5].ptr, (float *)b[6].ptr, (_Float16 *)b[7].ptr,
        (_Float16 *)b[8].ptr, (uint32_t)rows, p.pos, rope_frequencies(p.theta), p.eps);
    return nullptr;
}

const char *launch_batch_rope_half(Context &c, const View *b, int count, const boot_kernel_args &p, const uint32_t *) {
    // bindings (Prefill.cs:258 with Flags = KvFlags): q, k, v, qr, kc, vc; FP16 storage only (flags bit 256)
    BOOT_REQUIRE(count >= 6, "batch_rope needs 6 bindings: q, k, v, qr, kc, vc");
    BOOT_REQUIRE(p.flags & 256, "batch_rope serves the FP16 KV storage (flags bit 256); FP32 storage is not built");
    const uint64_t rows = p.m, end = (uint64_t)p.pos + rows;
    if (rows == 0) return nullptr;
    BOOT_REQUIRE(b[0].bytes >= rows * 16384 && b[3].bytes >= rows * 16384, "Q/rotated buffers smaller than rows*4096 floats");
    BOOT_REQUIRE(b[1].bytes >= rows * 2048 && b[2].bytes >= rows * 2048, "K/V input smaller than rows*512 floats");
    BOOT_REQUIRE(b[4].bytes >= end * 1024 && b[5].bytes >= end * 1024, "FP16 KV cache smaller than position+rows");
    BOOT_REQUIRE(aligned(b[0].ptr, 16) && aligned(b[1].ptr, 16) && aligned(b[2].ptr, 16) && aligned(b[3].ptr, 16) &&
                     aligned(b[4].ptr, 8) && aligned(b[5].ptr, 8),
                 "bindings misaligned");
    launch_timed(c, "batch_rope_half_kernel", batch_rope_half_kernel, dim3((uint32_t)((rows + 3) / 4)), dim3(256), 
        (const float *)b[0].ptr, (const float *)b[1].ptr, (const float *)b[2].ptr, (float *)b[3].ptr,
        (_Float16 *)b[4].ptr, (_Float16 *)b[5].ptr, (uint32_t)rows, p.pos, rope_frequencies(p.theta));
    return nullptr;
}

const char *launch_rmsnorm(Context &c, const View *b, int count, const boot_kernel_args &p, const uint32_t *) {
    // bindings (QwenEngine.cs:119): x, w (bf16), y, gate; N = 256, M groups, Epsilon, Flags (1: w+1, 2: silu gate)
    BOOT_REQUIRE(count >= 4, "rmsnorm needs 4 bindings: x, w, y, gate");
    BOOT_REQUIRE(p.n == 256, "rmsnorm serves the 256-wide head norms of the attention path");
    const uint64_t groups = p.m;
    if (groups == 0) return nullptr;
    BOOT_REQUIRE(b[0].bytes >= groups * 1024 && b[2].bytes >= groups * 1024, "x/y smaller than M*256 floats");
    BOOT_REQUIRE(b[1].bytes >= 512, "weights smaller than 256 bf16");
    BOOT_REQUIRE(!(p.flags & 2) || b[3].bytes >= groups * 1024, "gate smaller than M*256 floats");
    BOOT_REQUIRE(aligned(b[0].ptr, 16) && aligned(b[1].ptr, 8) && aligned(b[2].ptr, 16) && aligned(b[3].ptr, 16),
                 "bindings misaligned");
    rmsnorm256_kernel<<<(uint32_t)((groups + 3) / 4), 256, 0, context_stream(c)>>>(
        (const float *)b[0].ptr, (const uint16_t *)b[1].ptr, (float *)b[2].ptr, (const float *)b[3].ptr,
        (uint32_t)groups, p.eps, p.flags);
    return nullptr;
}

const char *launch_batch_split_q(Context &c, const View *b, int count, const boot_kernel_args &p, const uint32_t *) {
    // bindings (Prefill.cs:255): x [rows][8192], q [rows][4096], gate [rows][4096]
    BOOT_REQUIRE(count >= 3, "batch_split_q needs 3 bindings: x, q, gate");
    const uint64_t rows = p.m;
    if (rows == 0) return nullptr;
    BOOT_REQUIRE(b[0].bytes >= rows * 32768 && b[1].bytes >= rows * 16384 && b[2].bytes >= rows * 16384,
                 "buffers smaller than the split");
    BOOT_REQUIRE(aligned(b[0].ptr, 16) && aligned(b[1].ptr, 16) && aligned(b[2].ptr, 16), "bindings misaligned");
    const uint64_t threads = rows * 1024;
    batch_split_q_kernel<<<(uint32_t)((threads + 255) / 256), 256, 0, context_stream(c)>>>(
        (const float *)b[0].ptr, (float *)b[1].ptr, (float *)b[2].ptr, (uint32_t)rows);
    return nullptr;
}

hipError_t fill_zero(void *ptr, uint64_t bytes, hipStream_t stream) {
    if (bytes == 0) return hipSuccess;
    uintptr_t a = reinterpret_cast<uintptr_t>(ptr);
    if (a & 15) return hipErrorInvalidValue;  // buffers come from hipMalloc (256-byte aligned)
    const uint64_t n16 = bytes / 16;
    const uint32_t ntail = (uint32_t)(bytes % 16);
    uint64_t blocks = (n16 + 255) / 256;
    if (blocks > 8192) blocks = 8192;
    if (blocks == 0) blocks = 1;
    fill_zero_kernel<<<(uint32_t)blocks, 256, 0, stream>>>((uint4 *)ptr, n16, (uint8_t *)ptr + n16 * 16, ntail);
    return hipGetLastError();
}

}  // namespace boot
