// Device arithmetic shared by the append kernels and the fused decode+append: the wave
// reductions, the bit-exact INT8 quantizer (kernels.metal:135-140), the partial RoPE
// (kernels.metal:122-125) and the RMS norm of the fused preparation. One definition, so every
// kernel that rotates or quantizes a vector produces the same bits.
#pragma once
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

namespace boot {

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

// Rotation angles of one position for the four dims a lane holds (4*lane .. +3):
// lane j < 32 evaluates cos/sin of position * theta^(-2j/64) once
// (kernels.metal:122-125), and lanes fetch the pairs of their dims
// (j = d % 32) by shuffle, so one sincos per pair serves every head. `ifreq` is
// the lane's theta^(-2j/64) from lane_inv_freq.
struct Rope4 {
    float c[4], s[4];
};

__device__ inline Rope4 rope_angles(uint32_t position, int lane, float ifreq) {
    float cj = 1.0f, sj = 0.0f;
    if (lane < 32) {
        const float angle = (float)position * ifreq;
        sincosf(angle, &sj, &cj);
    }
    Rope4 r;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int j = (lane * 4 + i) & 31;
        r.c[i] = __shfl(cj, j, 64);
        r.s[i] = __shfl(sj, j, 64);
    }
    return r;
}

// Partial RoPE of the float4 a lane holds (dims 4*lane .. 4*lane+3) of one
// 256-dim head vector; dims < 64 rotate in pairs (j, j+32). The pair partner
// of lane l < 16 is lane l ^ 8. Every lane must call this (shuffles).
__device__ inline float4 rope4(float4 x, int lane, const Rope4 &r) {
    float4 p;
    p.x = __shfl_xor(x.x, 8, 64);
    p.y = __shfl_xor(x.y, 8, 64);
    p.z = __shfl_xor(x.z, 8, 64);
    p.w = __shfl_xor(x.w, 8, 64);
    if (lane >= 16) return x;
    float in[4] = {x.x, x.y, x.z, x.w}, partner[4] = {p.x, p.y, p.z, p.w}, out[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int d = lane * 4 + i;
        if (d < 32) out[i] = fmaf(in[i], r.c[i], -(partner[i] * r.s[i]));   // a*cos - b*sin, b = x[j+32]
        else out[i] = fmaf(in[i], r.c[i], partner[i] * r.s[i]);              // b*cos + a*sin, a = x[j]
    }
    return make_float4(out[0], out[1], out[2], out[3]);
}

// The 32 RoPE frequencies pow(theta, -float(2*j)/64.0f) of kernels.metal:123 as FP32 values,
// evaluated in FP64 and rounded once on the host for each dispatch (rope_frequencies), so each
// is the correctly rounded FP32 value of the reference's expression (theta and the exponent are
// exact in FP32); one ulp of one of them moves the angle at position 262143 by ~0.016 rad. Every
// kernel that rotates takes them from here, so all of them rotate with identical bits.
struct RopeFreq {
    float f[32];
};

__host__ inline RopeFreq rope_frequencies(float theta) {
    RopeFreq t;
    for (int j = 0; j < 32; j++) t.f[j] = (float)pow((double)theta, (double)(-(float)(2 * j) / 64.0f));
    return t;
}

// Lane j < 32 of the wave gets frequency j (selected from the kernel argument's scalar values,
// no memory access per lane); lanes 32..63 get 0.
__device__ inline float lane_inv_freq(const RopeFreq &t) {
    const int lane = threadIdx.x & 63;
    float r = 0.0f;
#pragma unroll
    for (int j = 0; j < 32; j++) r = lane == j ? t.f[j] : r;
    return r;
}

// RMS normalization of one 256-dim vector held as a float4 per lane, with the
// weights (bf16 w + 1) of QwenEngine's q_norm/k_norm (kernels.metal:51-57 with
// flag 1): y = x * (1/sqrt(mean(x^2) + eps)) * (w + 1). The sum of squares
// has one fixed order (lane partial, then a butterfly), shared by rmsnorm and
// the fused preparation so both give identical bits.
__device__ inline float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

__device__ inline float bf16_to_float(uint16_t b) { return __builtin_bit_cast(float, (uint32_t)b << 16); }

__device__ inline float4 rms_norm4(float4 x, float eps, const uint16_t *w, int lane, float offset) {
    const float total = wave_sum(((x.x * x.x + x.y * x.y) + x.z * x.z) + x.w * x.w);
    const float inv = 1.0f / sqrtf(total / 256.0f + eps);
    const uint2 wb = *reinterpret_cast<const uint2 *>(w + 4 * lane);
    float4 y;
    y.x = x.x * inv * (bf16_to_float(wb.x & 0xffff) + offset);
    y.y = x.y * inv * (bf16_to_float(wb.x >> 16) + offset);
    y.z = x.z * inv * (bf16_to_float(wb.y & 0xffff) + offset);
    y.w = x.w * inv * (bf16_to_float(wb.y >> 16) + offset);
    return y;
}

struct KNorm {
    const uint16_t *w;   // k_norm weights (bf16); null: no normalization
    float eps;
};

}  // namespace boot
