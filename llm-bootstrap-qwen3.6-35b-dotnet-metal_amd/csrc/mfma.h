// gfx950 MFMA operand types and INT8 -> FP16/BF16 register dequantization.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace boot {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

// Four signed INT8 codes -> four FP16 values, exactly. Bytes are biased to
// unsigned (x ^ 0x80), placed under the FP16 exponent of 1024 (0x64XX is
// 1024 + XX), and 1152 = 1024 + 128 is subtracted in packed FP16; every step
// is exact for |code| <= 128.
__device__ inline void i8x4_to_f16(uint32_t w, uint32_t &lo, uint32_t &hi) {
    const uint32_t u = w ^ 0x80808080u;
    uint32_t a = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);
    uint32_t b = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);
    half2v ha = __builtin_bit_cast(half2v, a), hb = __builtin_bit_cast(half2v, b);
    const half2v bias = {(_Float16)1152.0f, (_Float16)1152.0f};
    ha -= bias;
    hb -= bias;
    lo = __builtin_bit_cast(uint32_t, ha);
    hi = __builtin_bit_cast(uint32_t, hb);
}

// The same conversion in four instructions: each converts one byte, sign-extended by the
// operand select (SDWA), from INT16 to FP16 and writes one half of its destination, the
// second write of a destination keeping the half the first wrote. The two destinations
// alternate, so no instruction reads a register its direct predecessor wrote with a half
// select (a dst_sel result may reach the next VALU unshifted). Volatile, so that it keeps
// its place among the assembly MFMAs. Exact: every INT8 value is an FP16 integer.
__device__ inline void i8x4_to_f16_sdwa(uint32_t w, uint32_t &lo, uint32_t &hi) {
    asm volatile(
        "v_cvt_f16_i16_sdwa %0, sext(%2) dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:BYTE_0\n\t"
        "v_cvt_f16_i16_sdwa %1, sext(%2) dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:BYTE_2\n\t"
        "v_cvt_f16_i16_sdwa %0, sext(%2) dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:BYTE_1\n\t"
        "v_cvt_f16_i16_sdwa %1, sext(%2) dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:BYTE_3"
        : "=&v"(lo), "=&v"(hi)
        : "v"(w));
}

// The same conversion in two halves, for code that spreads it over several places: _lo writes
// bytes 0 and 2 into the low halves of lo and hi, _hi bytes 1 and 3 into their high halves
// (keeping the low ones). Between the two, lo and hi hold half-written words.
__device__ inline void i8x4_to_f16_sdwa_lo(uint32_t w, uint32_t &lo, uint32_t &hi) {
    asm volatile(
        "v_cvt_f16_i16_sdwa %0, sext(%2) dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:BYTE_0\n\t"
        "v_cvt_f16_i16_sdwa %1, sext(%2) dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:BYTE_2"
        : "=&v"(lo), "=&v"(hi)
        : "v"(w));
}
__device__ inline void i8x4_to_f16_sdwa_hi(uint32_t w, uint32_t &lo, uint32_t &hi) {
    asm volatile(
        "v_cvt_f16_i16_sdwa %0, sext(%2) dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:BYTE_1\n\t"
        "v_cvt_f16_i16_sdwa %1, sext(%2) dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:BYTE_3"
        : "+v"(lo), "+v"(hi)
        : "v"(w));
}

// Eight codes (two dwords) in eight SDWA conversions, not volatile: where the order among
// assembly MFMAs does not matter, the compiler schedules them freely (the decode's PV: against the
// perm-and-subtract form, 10 instructions per 8 codes, 28.9-29.0 against 29.2-29.4 us per layer
// step). Each word is written low half first; a register's high-half write is four instructions
// after its low-half write, never right behind it.
__device__ inline void i8x8_to_f16_sdwa(uint32_t w0, uint32_t w1, uint32_t &h0, uint32_t &h1, uint32_t &h2,
                                        uint32_t &h3) {
    asm("v_cvt_f16_i16_sdwa %0, sext(%4) dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:BYTE_0\n\t"
        "v_cvt_f16_i16_sdwa %1, sext(%4) dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:BYTE_2\n\t"
        "v_cvt_f16_i16_sdwa %2, sext(%5) dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:BYTE_0\n\t"
        "v_cvt_f16_i16_sdwa %3, sext(%5) dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:BYTE_2\n\t"
        "v_cvt_f16_i16_sdwa %0, sext(%4) dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:BYTE_1\n\t"
        "v_cvt_f16_i16_sdwa %1, sext(%4) dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:BYTE_3\n\t"
        "v_cvt_f16_i16_sdwa %2, sext(%5) dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:BYTE_1\n\t"
        "v_cvt_f16_i16_sdwa %3, sext(%5) dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:BYTE_3"
        : "=&v"(h0), "=&v"(h1), "=&v"(h2), "=&v"(h3)
        : "v"(w0), "v"(w1));
}

// Eight INT8 codes (two dwords) -> half8 operand, in byte order.
__device__ inline half8 i8x8_to_half8(uint32_t w0, uint32_t w1) {
    uint32_t r[4];
    i8x4_to_f16(w0, r[0], r[1]);
    i8x4_to_f16(w1, r[2], r[3]);
    return __builtin_bit_cast(half8, *reinterpret_cast<uint4 *>(r));
}

// Four signed INT8 codes -> four BF16 values, exactly: the FP16 integers are
// converted through FP32 (exact) and truncated to BF16 (exact for |code| <= 256).
__device__ inline void i8x4_to_bf16(uint32_t w, uint32_t &lo, uint32_t &hi) {
    const float f0 = (float)(int8_t)(w & 0xff), f1 = (float)(int8_t)((w >> 8) & 0xff);
    const float f2 = (float)(int8_t)((w >> 16) & 0xff), f3 = (float)(int8_t)(w >> 24);
    lo = (__builtin_bit_cast(uint32_t, f0) >> 16) | (__builtin_bit_cast(uint32_t, f1) & 0xffff0000u);
    hi = (__builtin_bit_cast(uint32_t, f2) >> 16) | (__builtin_bit_cast(uint32_t, f3) & 0xffff0000u);
}

__device__ inline bf16x8 i8x8_to_bf16x8(uint32_t w0, uint32_t w1) {
    uint32_t r[4];
    i8x4_to_bf16(w0, r[0], r[1]);
    i8x4_to_bf16(w1, r[2], r[3]);
    return __builtin_bit_cast(bf16x8, *reinterpret_cast<uint4 *>(r));
}

// FP32 -> BF16 bits, round to nearest even (finite inputs).
__device__ inline uint32_t bf16_bits(float x) {
    uint32_t u = __builtin_bit_cast(uint32_t, x);
    return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}

__device__ inline float bf16_value(uint32_t bits) { return __builtin_bit_cast(float, bits << 16); }

}  // namespace boot
