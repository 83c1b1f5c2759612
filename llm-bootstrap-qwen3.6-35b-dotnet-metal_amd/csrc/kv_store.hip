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

namespace boot {
namespace {

constexpr int kTile = 64;               // tokens per store work-group (page-aligned tiles)
constexpr int kVtStride = 68;           // bytes per LDS row of the V transpose (17 dwords)

__device__ inline float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

__device__ inline float quant_code(float x, float amax, float recip) {
    // kernels.metal:140: clamp(rint(amax > 0 ? x * (127/amax) : 0), -127, 127)
    float c = amax > 0.0f ? rintf(x * recip) : 0.0f;
    return fminf(fmaxf(c, -127.0f), 127.0f);
}

__device__ inline uint32_t pack4(float a, float b, float c, float d) {
    return (uint32_t)(uint8_t)(int8_t)(int)a | ((uint32_t)(uint8_t)(int8_t)(int)b << 8) |
           ((uint32_t)(uint8_t)(int8_t)(int)c << 16) | ((uint32_t)(uint8_t)(int8_t)(int)d << 24);
}

// Partial RoPE of the float4 a lane holds (dims 4*lane .. 4*lane+3) of one
// 256-dim head vector; dims < 64 rotate in pairs (j, j+32), j = d % 32,
// angle = position * theta^(-2j/64) (kernels.metal:122-125). The pair partner
// of lane l < 16 is lane l ^ 8. Every lane must call this (shuffles).
__device__ inline float4 rope4(float4 x, int lane, uint32_t position, const float *inv_freq) {
    float4 p;
    p.x = __shfl_xor(x.x, 8, 64);
    p.y = __shfl_xor(x.y, 8, 64);
    p.z = __shfl_xor(x.z, 8, 64);
    p.w = __shfl_xor(x.w, 8, 64);
    if (lane >= 16) return x;
    float in[4] = {x.x, x.y, x.z, x.w}, partner[4] = {p.x, p.y, p.z, p.w}, out[4];
    const float fpos = (float)position;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        int d = lane * 4 + i, j = d & 31;
        float angle = fpos * inv_freq[j];
        float c = cosf(angle), s = sinf(angle);
        if (d < 32) out[i] = fmaf(in[i], c, -(partner[i] * s));   // a*cos - b*sin, b = x[j+32]
        else out[i] = fmaf(in[i], c, partner[i] * s);              // b*cos + a*sin, a = x[j]
    }
    return make_float4(out[0], out[1], out[2], out[3]);
}

__device__ inline void fill_inv_freq(float *inv_freq, float theta) {
    // pow(theta, -float(2*j)/64.0f) in fp32, kernels.metal:123
    if (threadIdx.x < 32) inv_freq[threadIdx.x] = powf(theta, -(float)(2 * threadIdx.x) / 64.0f);
}

// Quantizes and appends tokens [lo, hi) of one 64-token tile for one KV head.
// K: one wave per token, float4 per lane, codes written token-major as char4.
// V: codes transposed in LDS, then written as page rows (16-byte stores for a
// full tile, byte stores at partial tile edges), kernels.metal:126-128.
template <bool Rope>
__device__ void store_tile(const float *__restrict__ k, const float *__restrict__ v,
                           int8_t *__restrict__ kc, int8_t *__restrict__ vc,
                           float *__restrict__ ks, float *__restrict__ vs,
                           uint32_t rows, uint32_t pos, uint32_t tile, uint32_t h,
                           uint8_t *vt, const float *inv_freq) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t tile0 = tile * kTile;
    const uint32_t lo = max(tile0, pos), hi = min(tile0 + kTile, pos + rows);
    for (uint32_t tl = wave; tl < kTile; tl += 4) {
        const uint32_t t = tile0 + tl;
        if (t < lo || t >= hi) continue;  // wave-uniform
        const uint32_t row = t - pos;
        const float *kr = k + ((size_t)row * 2 + h) * 256;
        const float *vr = v + ((size_t)row * 2 + h) * 256;
        float4 kx = *reinterpret_cast<const float4 *>(kr + 4 * lane);
        float vx0 = vr[lane], vx1 = vr[lane + 64], vx2 = vr[lane + 128], vx3 = vr[lane + 192];
        if (Rope) kx = rope4(kx, lane, t, inv_freq);
        float ka = wave_max(fmaxf(fmaxf(fabsf(kx.x), fabsf(kx.y)), fmaxf(fabsf(kx.z), fabsf(kx.w))));
        float va = wave_max(fmaxf(fmaxf(fabsf(vx0), fabsf(vx1)), fmaxf(fabsf(vx2), fabsf(vx3))));
        const uint64_t vector = (uint64_t)t * 2 + h;
        if (lane == 0) {
            ks[vector] = ka / 127.0f;
            vs[vector] = va / 127.0f;
        }
        const float kr127 = 127.0f / ka, vr127 = 127.0f / va;
        *reinterpret_cast<uint32_t *>(kc + vector * 256 + 4 * lane) =
            pack4(quant_code(kx.x, ka, kr127), quant_code(kx.y, ka, kr127),
                  quant_code(kx.z, ka, kr127), quant_code(kx.w, ka, kr127));
        vt[(lane + 0) * kVtStride + tl] = (uint8_t)(int8_t)(int)quant_code(vx0, va, vr127);
        vt[(lane + 64) * kVtStride + tl] = (uint8_t)(int8_t)(int)quant_code(vx1, va, vr127);
        vt[(lane + 128) * kVtStride + tl] = (uint8_t)(int8_t)(int)quant_code(vx2, va, vr127);
        vt[(lane + 192) * kVtStride + tl] = (uint8_t)(int8_t)(int)quant_code(vx3, va, vr127);
    }
    __syncthreads();
    const uint64_t base = ((uint64_t)(tile0 >> 8) * 2 + h) * kPageBytes + (tile0 & 255);
    if (lo == tile0 && hi == tile0 + kTile) {
        for (int item = threadIdx.x; item < 256 * 4; item += 256) {
            const int d = item >> 2, s = item & 3;
            const uint32_t *src = reinterpret_cast<const uint32_t *>(vt + d * kVtStride + s * 16);
            *reinterpret_cast<uint4 *>(vc + base + (uint64_t)d * 256 + s * 16) =
                make_uint4(src[0], src[1], src[2], src[3]);
        }
    } else {
        for (int item = threadIdx.x; item < 256 * kTile; item += 256) {
            const int d = item >> 6, tl = item & 63;
            const uint32_t t = tile0 + tl;
            if (t >= lo && t < hi) vc[base + (uint64_t)d * 256 + tl] = vt[d * kVtStride + tl];
        }
    }
}

__global__ __launch_bounds__(256) void kv_store_int8_kernel(
    const float *__restrict__ k, const float *__restrict__ v, int8_t *__restrict__ kc,
    int8_t *__restrict__ vc, float *__restrict__ ks, float *__restrict__ vs, uint32_t rows,
    uint32_t pos, uint32_t first_tile) {
    __shared__ __attribute__((aligned(16))) uint8_t vt[256 * kVtStride];
    store_tile<false>(k, v, kc, vc, ks, vs, rows, pos, first_tile + blockIdx.x / 2, blockIdx.x & 1,
                      vt, nullptr);
}

// batch_rope_int8 (kernels.metal:142-146): blocks [0, qblocks) rotate the
// 16 query heads of every row into qr; the remaining blocks rotate K and
// append K/V tiles. One launch.
__global__ __launch_bounds__(256) void batch_rope_int8_kernel(
    const float *__restrict__ q, const float *__restrict__ k, const float *__restrict__ v,
    float *__restrict__ qr, int8_t *__restrict__ kc, int8_t *__restrict__ vc,
    float *__restrict__ ks, float *__restrict__ vs, uint32_t rows, uint32_t pos, float theta,
    uint32_t qblocks, uint32_t first_tile) {
    __shared__ __attribute__((aligned(16))) uint8_t vt[256 * kVtStride];
    __shared__ float inv_freq[32];
    fill_inv_freq(inv_freq, theta);
    __syncthreads();
    if (blockIdx.x < qblocks) {
        const int lane = threadIdx.x & 63;
        const uint32_t vec = blockIdx.x * 4 + (threadIdx.x >> 6);   // row*16 + head
        if (vec >= rows * 16) return;                                // wave-uniform
        const uint32_t row = vec / 16;
        float4 x = *reinterpret_cast<const float4 *>(q + (size_t)vec * 256 + 4 * lane);
        x = rope4(x, lane, pos + row, inv_freq);
        *reinterpret_cast<float4 *>(qr + (size_t)vec * 256 + 4 * lane) = x;
        return;
    }
    const uint32_t b = blockIdx.x - qblocks;
    store_tile<true>(k, v, kc, vc, ks, vs, rows, pos, first_tile + b / 2, b & 1, vt, inv_freq);
}

__global__ __launch_bounds__(256) void query_grouped_half_kernel(const float *__restrict__ x,
                                                                 _Float16 *__restrict__ y,
                                                                 uint32_t rows, uint32_t group) {
    // kernels.metal:1276-1281, four values per thread
    const uint64_t at = ((uint64_t)blockIdx.x * 256 + threadIdx.x) * 4;
    if (at >= (uint64_t)rows * 4096) return;
    const uint64_t d = at % 256, logical = at / 256, span = (uint64_t)rows * group;
    const uint64_t block = logical / span, local = logical % span;
    const uint64_t row = local / group, head = block * group + local % group;
    const float4 v = *reinterpret_cast<const float4 *>(x + (row * 16 + head) * 256 + d);
    typedef _Float16 half4 __attribute__((ext_vector_type(4)));
    half4 o = {(_Float16)v.x, (_Float16)v.y, (_Float16)v.z, (_Float16)v.w};   // RNE
    *reinterpret_cast<half4 *>(y + at) = o;
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
    const uint32_t first = p.pos / kTile, last = (uint32_t)((end - 1) / kTile);
    const uint32_t blocks = (last - first + 1) * 2;
    kv_store_int8_kernel<<<blocks, 256, 0, context_stream(c)>>>(
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
    const uint32_t qblocks = (uint32_t)((rows * 16 + 3) / 4);
    const uint32_t first = p.pos / kTile, last = (uint32_t)((end - 1) / kTile);
    const uint32_t blocks = qblocks + (last - first + 1) * 2;
    batch_rope_int8_kernel<<<blocks, 256, 0, context_stream(c)>>>(
        (const float *)b[0].ptr, (const float *)b[1].ptr, (const float *)b[2].ptr, (float *)b[3].ptr,
        (int8_t *)b[4].ptr, (int8_t *)b[5].ptr, (float *)b[6].ptr, (float *)b[7].ptr, (uint32_t)rows,
        p.pos, p.theta, qblocks, first);
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
    BOOT_REQUIRE(aligned(b[0].ptr, 16) && aligned(b[1].ptr, 8), "query bindings misaligned");
    const uint64_t threads = rows * 1024;
    query_grouped_half_kernel<<<(uint32_t)((threads + 255) / 256), 256, 0, context_stream(c)>>>(
        (const float *)b[0].ptr, (_Float16 *)b[1].ptr, (uint32_t)rows, p.a);
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
