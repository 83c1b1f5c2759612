// Causal online GQA prefill over the INT8 KV cache (block prefill, <= 512-token
// chunks), MFMA on gfx950, and the FP16-KV control on the same schedule.
//
// Reference semantics: attention_int8_prefill / attention_online_int8_q32_k256_r2
// (kernels.metal:1378-1457), dispatched by DeviceAttentionWorkspace.EncodeInt8
// (DeviceAttention.cs:65-70):
//   s[r][t] = (q16[r] . kcode[t]) * (1/16) * ks[t]        FP16 Q x INT8 K, FP32 accumulate
//   online max / sum over t <= pos + r/8 (FP32 statistics, l sums unscaled e)
//   P[r][t] = bf16(e * vs[t]);  o = o * decay + P . vcode  BF16 x INT8 V, FP32 accumulate
//   y = o / l * sigmoid(gate)
// One deliberate change: the scaled probabilities are rounded to FP16 after
// dividing the V scales by their maximum over the work-group's key range
// (vs_ref) and multiplying them by 2^7, and vs_ref / 2^7 multiplies the result
// once at the end. e * 2^7 * vs / vs_ref lies in [0, 2^15], so FP16 neither
// overflows nor drops small probabilities into its subnormals (the reason the
// reference chose BF16, docs/INT8_KV_20261104.md:16), and its rounding is 8x
// finer than BF16's. The denominator sums the rounded operands divided back by
// their factor (P / (2^7 vs / vs_ref), one mixed FP16 x FP32 FMA per element in
// place of the add of e), so an operand's rounding moves numerator and
// denominator together: a row dominated by one key returns that key's value
// exactly, and the remaining error scales with the spread of the values, not
// their size (heavy-tailed V reaches |y| ~ 16, where a denominator of unrounded
// e leaves FP16's relative 2^-12 as an absolute error above 2e-3).
// Logical row r of KV group g is (token r/8, head 8g + r%8): the grouped FP16
// query layout of attention_query_grouped_half (kernels.metal:1276-1281).
// The FP16-KV control (attention_online_q32_k256_s8_g8_r2, kernels.metal:1356-1365:
// FP16 token-major K and V, no scales) runs the same kernel with FP16 staging, so that
// the two differ only in the cache they read.
//
// gfx950 structure (not the Metal tiling): S^T = K . Q^T and O^T += V^T . P^T with
// v_mfma_f32_32x32x16_f16 on FP16 operands staged in LDS (INT8 codes are exact in
// FP16). Transposed products put one query row per lane column, so row statistics
// are per-lane and the accumulator rescale needs no cross-lane traffic; the key
// order inside each QK tile is permuted so a lane's S registers are exactly its
// FP16 B operand for the PV product. The exponentials run in the base-2 domain
// (the K scale carries log2(e)/16) against a lazy running maximum. Long histories
// split the key range across work-groups (split-K) and a combine kernel merges
// (m, l, O); the splits of a row tile are placed on one XCD, so that its L2 holds
// the tile's query for all of them and their partials for the combine.
#include "common.h"
#include <type_traits>
#include "mfma.h"

namespace boot {

namespace {

constexpr int kKStride = 256 + 8;          // FP16 K tile row stride (halves): 528 bytes
constexpr float kLog2e = 1.4426950408889634f;
constexpr int kTileRows = 256;             // logical rows per work-group (32 tokens x 8 heads)
// Split partial of one work-group: O^T / l per row in region A ([256 rows][512 B]: the row in FP16,
// or dimensions 0-127 in FP32) and region B (dimensions 128-255 of FP32 rows; the epilogue chooses
// the format per row), then m, l and vs_ref / 2^7 per row as floats, the last negated for FP32
// rows. FP16 rows, the common case, are as compact as a plain FP16 partial.
constexpr size_t kPartialRegion = (size_t)kTileRows * 512;
constexpr size_t kPartialBytes = 2 * kPartialRegion + 3 * kTileRows * 4;
// A row's partial is FP16 when its outputs are at most this large (FP16's relative 2^-12 of 4 is
// 9.8e-4), FP32 otherwise.
constexpr float kNarrowPartial = 4.0f;
// Prefill chunks of at most 64 rows with rows x keys up to this go through the decode kernel.
constexpr uint64_t kDecodeRouteWork = 65536;

struct PrefillParams {
    const _Float16 *q;      // grouped FP16 [2][M][8][256]
    const void *k;          // INT8 [cap][2][256] codes, or FP16 [cap][2][256] (control)
    const void *v;          // INT8 V pages, or FP16 token-major [cap][2][256] (control)
    const float *gate;      // [M][16][256]
    float *y;               // [M][16][256]
    const float *ks, *vs;   // [cap][2]
    float *partial;         // split workspace
    uint32_t rows;          // M tokens in the chunk
    uint32_t pos;           // history
    uint32_t keys;          // K = pos + M
    uint32_t tiles;         // 256-row tiles per group
    uint32_t splits;
    uint32_t split_keys;    // multiple of the 32-key tile
    uint32_t remap;         // block order: 2 a row tile's splits on one XCD, 1 a key range's blocks on one XCD
};

// sigmoid(x) = 1 / (1 + 2^(-x log2(e))) with the hardware exponential and reciprocal (about an ulp
// each); a library expf and a correctly rounded division cost ~25 instructions per output element
__device__ inline float sigmoidf(float x) { return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-x * kLog2e)); }

// Key row of QK tile row i: bits 2 and 3 of i swapped (see header comment).
__device__ inline int qk_key_row(int i) { return (i & ~12) | ((i & 4) << 1) | ((i & 8) >> 1); }

// v_max3_f32 without the canonicalizing moves the compiler adds in front of
// fmaxf when it cannot prove its inputs canonical (no NaN reaches this kernel).
__device__ inline float max3f(float a, float b, float c) {
    float r;
    asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
    return r;
}

// Max over the lane pair (l, l ^ 32). v_permlane32_swap exchanges lanes 32-63 of
// its first operand with lanes 0-31 of its second, so with both holding x every
// lane ends with its own value in one register and its partner's in the other.
// Inline assembly: with the builtin, the compiler keeps only the first result when
// both operands are the same value, and the maximum then misses the partner lane.
// The no-ops cover the wait states around the cross-lane move.
__device__ inline float pair_max(float x) {
    float a = x, b = x;
    asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
    return max3f(a, b, b);
}


// S += A B^T with the accumulators in architectural VGPRs. At one wave per SIMD the compiler
// gives every MFMA of a kernel the accumulator-register form; where O already fills the 256
// accumulator registers, these keep S out of them. Dependent MFMAs of one chain (srcC exactly
// the previous destination, same opcode) need no wait states; the chain's last MFMA is followed
// by 24, which cover vector reads and writes of S after it (the 8-pass XDL RAW/WAW/WAR windows).
// The operands come from LDS or global loads (no VALU write precedes an MFMA read).
__device__ __forceinline__ void s_mfma_first(floatx16 &s, const half8 &a, const half8 &b) {
    asm volatile("v_mfma_f32_32x32x16_f16 %0, %1, %2, 0" : "=&v"(s) : "v"(a), "v"(b));
}
__device__ __forceinline__ void s_mfma(floatx16 &s, const half8 &a, const half8 &b) {
    asm volatile("v_mfma_f32_32x32x16_f16 %0, %1, %2, %0" : "+v"(s) : "v"(a), "v"(b));
}
__device__ __forceinline__ void s_mfma_last(floatx16 &s, const half8 &a, const half8 &b) {
    asm volatile("v_mfma_f32_32x32x16_f16 %0, %1, %2, %0\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7"
                 : "+v"(s)
                 : "v"(a), "v"(b));
}
// O += A B^T with O in accumulator registers, as assembly for the same reason as s_mfma: the
// compiler schedules its MFMAs freely and moves operand reads from LDS next to them, exposing
// their latency. Dependent MFMAs of one chain need no wait states (exact srcC overlap); a vector
// write of an operand (the FP16 P) precedes these by far more than the two wait states it needs
// (a work-group barrier and LDS reads lie between); accumulator reads after the chain (rescale,
// epilogue) are preceded by 24 wait states written beside them.
__device__ __forceinline__ void o_mfma(floatx16 &o, const half8 &a, const half8 &b) {
    asm volatile("v_mfma_f32_32x32x16_f16 %0, %1, %2, %0" : "+a"(o) : "v"(a), "v"(b));
}
// Orders vector work after an assembly MFMA: the registers named here pass through the statement
// unchanged, so their consumers cannot be scheduled ahead of it (the scheduler places an assembly
// statement's independent neighbours freely).
__device__ __forceinline__ void after_mfma(float &z, float &w) { asm volatile("" : "+v"(z), "+v"(w)); }
__device__ __forceinline__ void after_mfma(uint32_t &x, uint32_t &y, uint32_t &z, uint32_t &w) {
    asm volatile("" : "+v"(x), "+v"(y), "+v"(z), "+v"(w));
}
// The other side: values named here are computed before the next assembly MFMA (volatile
// assembly keeps its order), so that a step's vector work stays between its two MFMAs instead of
// collecting in long runs the matrix pipe waits through.
__device__ __forceinline__ void before_mfma(float x, float y) { asm volatile("" ::"v"(x), "v"(y)); }
__device__ __forceinline__ void before_mfma(float x, float y, uint32_t z) { asm volatile("" ::"v"(x), "v"(y), "v"(z)); }

// ---------------------------------------------------------------- prefill, one wave per SIMD
//
// A work-group of 4 waves (one per SIMD, up to 512 registers each) owns 256 logical rows of one
// KV group and walks its key range in 32-key tiles; wave w owns rows 64w .. 64w + 63 as two
// 32-row blocks, so every K or V operand read from LDS feeds two MFMAs, most of its query stays
// in registers and its O^T accumulators fill the accumulator registers. The wave overlaps its
// own vector work with its MFMAs: an MFMA occupies the matrix pipe for ~32 cycles while the wave
// issues independent VALU instructions beside it (about six per MFMA come free). Tile n runs in
// two phases, one work-group barrier apart:
//   A: S(n) = K(n) Q^T for both row blocks (32 MFMAs), interleaved with the exponentials of
//      tile n - 1 (P(n - 1), FP16, and l);
//   B: O += V(n - 1)^T P(n - 1) (32 MFMAs), interleaved with S(n)'s scaling and row maxima, the
//      staging of tile n + 2 (INT8: codes converted to FP16; FP16: copied, V transposed) and
//      the loads of tile n + 3.
// Rows whose maximum grows by more than 2^8, and tiles on the causal diagonal, take a fix-up
// after phase B (the general softmax); the common case needs no maximum before exp2. The
// MFMAs are inline assembly, so that their order, and the operand reads placed three steps
// ahead of them, are kept; each step's vector work is tied behind its MFMA. K tiles are
// double-buffered and V tiles (with the tile's scales) quadruple-buffered: every buffer a
// phase writes was last read before the previous barrier.
constexpr int kW64Keys = 32;               // keys per tile
// Lazy running maximum: a row rebases when a tile's maximum exceeds it by more than 2^kRebase
// (log2 units). Exponentials then stay <= 2^8, so P = e * 2^7 * vs / vs_ref (<= 2^15) is finite in
// FP16 (largest 65504); a maximum that lags only makes the kept exponentials larger.
constexpr float kRebase = 8.0f;
constexpr float kPScale = 128.0f;          // 2^7: the probability operand's factor (see above)
constexpr int kW64VBufs = 4;               // V^T tiles in LDS
// Q^T chunks per row block kept in LDS, the rest in registers (phase A reads the LDS ones two
// steps ahead). The INT8 kernel keeps twelve in registers: from nine to twelve, 3451 -> 3350
// cycles per tile with no spill (the probability factors and their reciprocals are read a key
// pair at a time, two steps ahead, so the row sums' reciprocals take no registers from them; read
// four keys at a time and four steps ahead they pushed a query chunk to scratch). The FP16
// control's staging holds more registers and spills beyond nine (3878 -> 4604 cycles with ten).
// At least four stay in LDS: the epilogue stages one wave's 32 KB of rows in that region.
template <bool kInt8>
constexpr int w64_qlds() { return kInt8 ? 4 : 7; }
#ifndef BOOT_W64_VAHEAD
#define BOOT_W64_VAHEAD 3
#endif
constexpr int kW64VAhead = BOOT_W64_VAHEAD;   // V operand reads in flight ahead of the PV MFMAs

struct W64KTile {
    _Float16 k[kW64Keys * kKStride];       // K codes as FP16, key-major (528-byte rows)
};
struct W64VTile {
    _Float16 v[256 * kW64Keys];            // V^T codes as FP16: 64-byte dimension rows whose 16-byte
                                           // pieces are XOR-swizzled by (row / 4) % 4
    float ks[kW64Keys];                    // K scale * log2(e) / 16 (0 beyond K)
    float4 rv[kW64Keys / 2];               // per key pair: r = 2^7 V scale / vs_ref (2^7 for a zero
                                           // vector) and 1 / r of each key, {r0, 1/r0, r1, 1/r1}
                                           // (0 beyond K)
};

template <bool kInt8>
__global__ __launch_bounds__(256, 1) void prefill_w64_kernel(PrefillParams p) {
    __shared__ W64KTile kbuf[2];
    __shared__ W64VTile vbuf[kW64VBufs];
    constexpr int kW64QLds = w64_qlds<kInt8>(), kW64QRegs = 16 - kW64QLds;
    __shared__ uint4 qlds[kW64QLds][2][256];   // [chunk][row block][thread]
    __shared__ float vs_partial[4];

    uint32_t g, tile, split;
    {
        const uint32_t b = blockIdx.x;
        uint32_t combo;
        if (p.remap == 2) {
            // work-groups are dealt to the 8 XCDs round-robin by block index: (group, tile) pair
            // j takes XCD j % 8 with all of its splits
            const uint32_t xcd = b % 8, idx = b / 8;
            const uint32_t pair = xcd + 8 * (idx / p.splits);
            split = idx % p.splits;
            g = pair % 2;
            tile = pair / 2;
            combo = g + 2 * split;
        } else if (p.remap) {
            const uint32_t xcd = b % 8, idx = b / 8;
            combo = xcd + 8 * (idx / p.tiles);
            tile = idx % p.tiles;
        } else {
            combo = b / p.tiles;
            tile = b % p.tiles;
        }
        g = combo % 2;
        split = combo / 2;
    }
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // uniform: wave-level branches stay scalar
    const int i = lane & 31, kk = lane >> 5;
    const uint32_t R = p.rows * 8;
    const uint32_t r0 = tile * kTileRows + 64 * wave;          // first row of this wave
    uint32_t my_row[2], limit[2];
    bool row_valid[2];
#pragma unroll
    for (int rb = 0; rb < 2; rb++) {
        my_row[rb] = r0 + 32 * rb + i;
        row_valid[rb] = my_row[rb] < R;
        limit[rb] = p.pos + (row_valid[rb] ? my_row[rb] : R - 1) / 8;   // keys <= limit visible
    }
    const uint32_t tile_last = min(R - 1, tile * kTileRows + kTileRows - 1);
    const uint32_t tile_end = p.pos + tile_last / 8 + 1;               // keys [0, tile_end)
    const uint32_t kbeg = split * p.split_keys;
    const uint32_t kend = min(tile_end, kbeg + p.split_keys);
    const int ntiles = kend > kbeg ? (int)((kend - kbeg + kW64Keys - 1) / kW64Keys) : 0;
    const uint32_t wave_min_limit = p.pos + min(R - 1, r0) / 8;
    const uint32_t last_key0 = kbeg + (uint32_t)max(ntiles - 1, 0) * kW64Keys;   // loads never go past it

    // ---- staging. INT8: thread t converts 32 K codes (rows krow0 and krow0 + 4, 16 codes at
    // 16 * kchunk; a load instruction reads four whole 256-byte rows) and the 32 V codes of page
    // row t (V pages are already dimension-major). FP16: thread t copies 16-byte pieces of K rows
    // 4 (t / 32) + j (piece t % 32; a load reads two whole 512-byte rows) and transposes a block of
    // 4 keys (4 (t / 32) + r) x 8 dimensions (8 (t % 32) + e) of the key-major V into V^T.
    const int krow0 = 8 * wave + (lane >> 4), kchunk = lane & 15;   // INT8 K
    const int fgroup = tid >> 5, fpiece = tid & 31;                 // FP16 K rows / V keys, piece
    struct Raw {
        uint4 w[8];    // INT8: K rows krow0, krow0 + 4, V page row t; FP16: 4 K pieces, 4 V keys
        float ks, vs;  // INT8: scales of key t % 32
    };
    // A tile's loads in three parts, so that phase B can reissue each as soon as the staging has
    // consumed its registers: the scales, the K codes (pieces 0-3), the V codes (pieces 4-7).
    // (key0: the tile's first key, at most last_key0)
    auto load_part = [&](Raw &r, uint32_t key0, int part) __attribute__((always_inline)) {
        // (byte offsets below 2^28 for the 262144-token window: 32-bit offsets from the bases)
        if constexpr (kInt8) {
            if (part == 0) {
                const uint32_t at = (min(key0 + (uint32_t)(tid & 31), p.keys - 1) * 2 + g) * 4;   // bytes
                r.ks = *reinterpret_cast<const float *>(reinterpret_cast<const char *>(p.ks) + at);
                r.vs = *reinterpret_cast<const float *>(reinterpret_cast<const char *>(p.vs) + at);
            } else if (part == 1) {
                const int8_t *kcodes = (const int8_t *)p.k;
                const uint32_t ka = min(key0 + (uint32_t)krow0, p.keys - 1), kb2 = min(key0 + (uint32_t)krow0 + 4, p.keys - 1);
                r.w[0] = *reinterpret_cast<const uint4 *>(kcodes + ((ka * 2 + g) * 256 + kchunk * 16));
                r.w[1] = *reinterpret_cast<const uint4 *>(kcodes + ((kb2 * 2 + g) * 256 + kchunk * 16));
            } else {
                const int8_t *vcodes = (const int8_t *)p.v;
                const uint32_t offv = (uint32_t)value_index((uint64_t)key0 * 2 + g, 0) + (uint32_t)tid * 256;
                r.w[2] = *reinterpret_cast<const uint4 *>(vcodes + offv);
                r.w[3] = *reinterpret_cast<const uint4 *>(vcodes + (offv + 16));
            }
        } else {
            // keys past K are clamped to K - 1: the cache beyond K (NaN padding) is never read
            const _Float16 *kh = (const _Float16 *)p.k, *vh = (const _Float16 *)p.v;
            if (part == 0) {
                r.ks = r.vs = 0.0f;
            } else {
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const uint32_t key = min(key0 + (uint32_t)(4 * fgroup + j), p.keys - 1);
                    if (part == 1)
                        r.w[j] = *reinterpret_cast<const uint4 *>(kh + ((key * 2 + g) * 256 + 8 * fpiece));
                    else
                        r.w[4 + j] = *reinterpret_cast<const uint4 *>(vh + ((key * 2 + g) * 256 + 8 * fpiece));
                }
            }
        }
    };
    auto load_raw = [&](uint32_t key0) __attribute__((always_inline)) {
        Raw r;   // (the order phase B issues them in: the waits in the loop count on it)
        key0 = min(key0, last_key0);
        load_part(r, key0, 0);
        load_part(r, key0, 1);
        load_part(r, key0, 2);
        return r;
    };
    float vs_inv = 0.0f;
    // Staging in pieces, so that phase B can spread them between its MFMAs. Piece j < 4 writes K
    // (INT8: 8 converted codes; FP16: a copied 16-byte piece), piece 4 <= j < 8 V (INT8: 8
    // converted codes; FP16: dimensions 2 (j - 4) and 2 (j - 4) + 1 of the 4 keys). Every wave
    // writes the tile's scales (the same values from each wave: lane l carries key l % 32).
    const int vsw_stage = (tid >> 2) & 3;
    auto piece_words = [&](const Raw &r, int j, uint32_t (&x)[4]) __attribute__((always_inline)) {
        if constexpr (kInt8) {
            const uint4 &w = r.w[j >> 1];
            x[0] = (j & 1) ? w.z : w.x;
            x[1] = (j & 1) ? w.w : w.y;
            x[2] = x[3] = 0;
        } else if (j < 4) {
            x[0] = r.w[j].x;
            x[1] = r.w[j].y;
            x[2] = r.w[j].z;
            x[3] = r.w[j].w;
        } else {
            const int d = j - 4;   // dword d of each key: dimensions 8 fpiece + 2d, + 1
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const uint4 &w = r.w[4 + k];
                x[k] = d == 0 ? w.x : d == 1 ? w.y : d == 2 ? w.z : w.w;
            }
        }
    };
    // INT8 piece j (8 converted codes): K rows for j < 4, V^T row t for j >= 4
    auto store_piece = [&](W64KTile &kb, W64VTile &vb, int j, const uint4 &h) __attribute__((always_inline)) {
        if (j < 4)
            *reinterpret_cast<uint4 *>(kb.k + (krow0 + 4 * (j >> 1)) * kKStride + kchunk * 16 + 8 * (j & 1)) = h;
        else
            *reinterpret_cast<uint4 *>(vb.v + tid * kW64Keys + 8 * ((j - 4) ^ vsw_stage)) = h;
    };
    auto stage_piece = [&](W64KTile &kb, W64VTile &vb, int j, const uint32_t (&x)[4]) __attribute__((always_inline)) {
        if constexpr (kInt8) {
            uint4 h;
            i8x4_to_f16_sdwa(x[0], h.x, h.y);
            i8x4_to_f16_sdwa(x[1], h.z, h.w);
            store_piece(kb, vb, j, h);
        } else if (j < 4) {
            *reinterpret_cast<uint4 *>(kb.k + (4 * fgroup + j) * kKStride + 8 * fpiece) = make_uint4(x[0], x[1], x[2], x[3]);
        } else {
            // keys 4 fgroup .. + 3 of V^T rows e and e + 1: 8 bytes each, in the 16-byte piece
            // fgroup / 2 (XOR-swizzled by the row as the operand reads expect)
            const int e = 8 * fpiece + 2 * (j - 4);
            const uint2 lo = make_uint2(__builtin_amdgcn_perm(x[1], x[0], 0x05040100u), __builtin_amdgcn_perm(x[3], x[2], 0x05040100u));
            const uint2 hi = make_uint2(__builtin_amdgcn_perm(x[1], x[0], 0x07060302u), __builtin_amdgcn_perm(x[3], x[2], 0x07060302u));
            *reinterpret_cast<uint2 *>(vb.v + e * kW64Keys + 8 * ((fgroup >> 1) ^ ((e >> 2) & 3)) + 4 * (fgroup & 1)) = lo;
            *reinterpret_cast<uint2 *>(vb.v + (e + 1) * kW64Keys + 8 * ((fgroup >> 1) ^ (((e + 1) >> 2) & 3)) + 4 * (fgroup & 1)) = hi;
        }
    };
    auto stage_scales = [&](W64VTile &vb, uint32_t key0, const Raw &r) __attribute__((always_inline)) {
        const int t = tid & 31;
        const bool inside = key0 + t < p.keys;   // poisoned tails beyond K never reach S or P
        if constexpr (kInt8) {
            float ks = r.ks, vs = r.vs;
            after_mfma(ks, vs);   // the products stay where the call is (not hoisted to the loads)
            vb.ks[t] = inside ? ks * (kLog2e / 16.0f) : 0.0f;
            // a zero V vector (codes 0, scale 0) keeps the factor 2^7: its key adds nothing to O but
            // its weight to the denominator
            const float r = vs > 0.0f ? vs * vs_inv * kPScale : kPScale;
            reinterpret_cast<float2 *>(vb.rv)[t] = inside ? make_float2(r, __builtin_amdgcn_rcpf(r)) : make_float2(0.0f, 0.0f);
        } else {
            vb.ks[t] = inside ? kLog2e / 16.0f : 0.0f;
            reinterpret_cast<float2 *>(vb.rv)[t] = inside ? make_float2(kPScale, 1.0f / kPScale) : make_float2(0.0f, 0.0f);
        }
    };
    auto stage = [&](W64KTile &kb, W64VTile &vb, uint32_t key0, const Raw &r) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < 8; j++) {
            uint32_t x[4];
            piece_words(r, j, x);
            stage_piece(kb, vb, j, x);
        }
        stage_scales(vb, key0, r);
    };

    // INT8: V(n + 1) is staged in phase A of tile n (its buffer's previous tile, n - 3, was last read
    // in phase B of tile n - 2, before the last barrier), K(n + 2) in phase B of tile n, so each
    // phase writes half of the tile's LDS (a CU takes LDS writes at a third of its read rate, and
    // a write holds its wave until then)
    constexpr bool kVinA = kInt8;
    // ---- prologue: the query, the V scales of the split (vs_ref), tile 0's codes. The query
    // chunks kept in LDS go first and straight into LDS (global_load_lds_dwordx4: lane l's 16
    // bytes to the wave's base in M0 + 16 l), holding no registers in flight. They are issued in
    // assembly, unseen by the compiler's counter bookkeeping: a compiler-issued LDS load makes it
    // wait for every load before each use of any of them, while these, the oldest, have simply
    // landed whenever a later load has (the counter counts in order). The V scales, the codes of
    // tiles 0 and 1, and the register chunks of the query follow, in the order of first use, so
    // that the V-scale maximum, its barrier and the staging run while the last of them are in
    // flight. (The empty assembly statements keep the compiler from reordering the groups.)
#pragma unroll
    for (int rb = 0; rb < 2; rb++) {
        const uint32_t rr = row_valid[rb] ? my_row[rb] : R - 1;
        const _Float16 *qrow = p.q + ((size_t)g * R + rr) * 256 + 8 * kk;
#pragma unroll
        for (int c = kW64QRegs; c < 16; c++) {
            const uint32_t lds = (uint32_t)(uintptr_t)&qlds[c - kW64QRegs][rb][64 * wave];   // wave-uniform
            uint32_t saved;
            asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %2, off\n\ts_mov_b32 m0, %0"
                         : "=&s"(saved)
                         : "s"(lds), "v"(qrow + 16 * c)
                         : "memory");
        }
    }
    float vsv[16];   // the V scales of the split's first 4096 keys
#pragma unroll
    for (int it = 0; it < 16; it++) {
        const uint32_t key = kbeg + tid + 256 * it;
        vsv[it] = kInt8 && key < kend ? p.vs[(size_t)key * 2 + g] : 0.0f;
    }
    asm volatile("" ::: "memory");
    const Raw raw0 = load_raw(kbeg), raw1 = load_raw(kbeg + kW64Keys);
    asm volatile("" ::: "memory");
    half8 qop[2][kW64QRegs];
#pragma unroll
    for (int rb = 0; rb < 2; rb++) {
        const uint32_t rr = row_valid[rb] ? my_row[rb] : R - 1;
        const _Float16 *qrow = p.q + ((size_t)g * R + rr) * 256 + 8 * kk;
#pragma unroll
        for (int c = 0; c < kW64QRegs; c++) qop[rb][c] = *reinterpret_cast<const half8 *>(qrow + 16 * c);
    }
    float vs_ref = kInt8 ? 0.0f : 1.0f;   // FP16 KV: no V scales
#pragma unroll
    for (int it = 0; it < 16; it++) vs_ref = fmaxf(vs_ref, vsv[it]);
    if (kInt8)   // the rest of the split, eight loads in flight per thread (not one round trip per key)
        for (uint32_t k0 = kbeg + tid + 4096; k0 < kend; k0 += 2048) {
            float v8[8];
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const uint32_t key = k0 + 256 * u;
                v8[u] = key < kend ? p.vs[(size_t)key * 2 + g] : 0.0f;
            }
#pragma unroll
            for (int u = 0; u < 8; u++) vs_ref = fmaxf(vs_ref, v8[u]);
        }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) vs_ref = fmaxf(vs_ref, __shfl_xor(vs_ref, o, 64));
    if (lane == 0) vs_partial[wave] = vs_ref;
    __syncthreads();
    vs_ref = fmaxf(fmaxf(vs_partial[0], vs_partial[1]), fmaxf(vs_partial[2], vs_partial[3]));
    vs_ref = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(uint32_t, vs_ref)));
    vs_inv = __builtin_bit_cast(
        float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(uint32_t, vs_ref > 0.0f ? 1.0f / vs_ref : 0.0f)));
    stage(kbuf[0], vbuf[0], kbeg, raw0);
    if constexpr (kVinA) {   // tile 1's V waits for phase A of tile 0
#pragma unroll
        for (int j = 0; j < 4; j++) {
            uint32_t x[4];
            piece_words(raw1, j, x);
            stage_piece(kbuf[1], vbuf[1], j, x);
        }
        stage_scales(vbuf[1], kbeg + kW64Keys, raw1);
    } else {
        stage(kbuf[1], vbuf[1], kbeg + kW64Keys, raw1);
    }
    // the query chunks are in their registers before the loop (a use here makes the compiler wait
    // for their loads once, instead of before their MFMAs on every tile)
#pragma unroll
    for (int rb = 0; rb < 2; rb++)
#pragma unroll
        for (int c = 0; c < kW64QRegs; c++) asm volatile("" ::"v"(qop[rb][c]));
    // staged in phase B of tile 0 (INT8: its K and scales; the V codes held are tile 1's)
    Raw raw;
    if constexpr (kVinA) {
        raw.w[2] = raw1.w[2];
        raw.w[3] = raw1.w[3];
        const uint32_t key = min(kbeg + 2 * kW64Keys, last_key0);
        load_part(raw, key, 0);
        load_part(raw, key, 1);
    } else {
        raw = load_raw(kbeg + 2 * kW64Keys);
    }
    {
        // "tile -1", whose zero probabilities the first PV multiplies: zero V^T codes and scales,
        // not NaN
        static_assert(sizeof(W64VTile) % 16 == 0, "whole 16-byte stores");
        uint4 *z = reinterpret_cast<uint4 *>(&vbuf[kW64VBufs - 1]);
        for (int e = tid; e < (int)(sizeof(W64VTile) / 16); e += 256) z[e] = make_uint4(0, 0, 0, 0);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // the query's LDS chunks have landed
    __syncthreads();

    floatx16 o[2][8];
#pragma unroll
    for (int rb = 0; rb < 2; rb++)
#pragma unroll
        for (int dt = 0; dt < 8; dt++)
#pragma unroll
            for (int v = 0; v < 16; v++) o[rb][dt][v] = 0.0f;
    float m[2] = {-INFINITY, -INFINITY}, l[2] = {0.0f, 0.0f};
    float thr[2] = {-INFINITY, -INFINITY};   // a row needs the general softmax when its tile maximum exceeds thr
    half8 pb[2][2];          // P(n - 1): [row block][16-key step]
#pragma unroll
    for (int rb = 0; rb < 2; rb++)
#pragma unroll
        for (int e = 0; e < 8; e++) pb[rb][0][e] = pb[rb][1][e] = (_Float16)0.0f;
    auto qop_at = [&](int rb, int c) __attribute__((always_inline)) {
        return c < kW64QRegs ? qop[rb][c < kW64QRegs ? c : 0]
                             : __builtin_bit_cast(half8, qlds[c < kW64QRegs ? 0 : c - kW64QRegs][rb][tid]);
    };

    // The loop addresses its buffers by byte offsets that rotate from tile to tile (K: tile n's at
    // kcur; V: tiles n - 1, n, n + 1, n + 2 at vm1, vc0, vc1, vc2), not by index arithmetic per tile.
    auto ktile = [&](uint32_t off) __attribute__((always_inline)) -> W64KTile & {
        return *reinterpret_cast<W64KTile *>(reinterpret_cast<unsigned char *>(kbuf) + off);
    };
    auto vtile = [&](uint32_t off) __attribute__((always_inline)) -> W64VTile & {
        return *reinterpret_cast<W64VTile *>(reinterpret_cast<unsigned char *>(vbuf) + off);
    };
    constexpr uint32_t kKT = sizeof(W64KTile), kVT = sizeof(W64VTile);
    uint32_t kcur = 0, vm1 = (kW64VBufs - 1) * kVT, vc0 = 0, vc1 = kVT, vc2 = 2 * kVT;   // tile 0

    // the K scales of a tile's keys, as the softmax lanes hold them (element v of a lane's S row:
    // key 16 (v / 8) + 8 kk + v % 8)
    auto load_scales = [&](uint32_t vo, float4 (&x4)[4]) __attribute__((always_inline)) {
        const float *src = vtile(vo).ks;
#pragma unroll
        for (int q4 = 0; q4 < 4; q4++)
            x4[q4] = *reinterpret_cast<const float4 *>(src + 16 * (q4 >> 1) + 8 * kk + 4 * (q4 & 1));
    };
    // the probability factors and their reciprocals of the key pair of elements v, v + 1 (v even):
    // {r(v), 1 / r(v), r(v + 1), 1 / r(v + 1)}
    auto load_rv = [&](uint32_t vo, int v) __attribute__((always_inline)) {
        return vtile(vo).rv[8 * (v >> 3) + 4 * kk + ((v & 7) >> 1)];
    };

    // The softmax of tile n - 1, finished in phase A of tile n: element v of row block rb of
    // exp2(S) (e, with S scaled and shifted by the running maximum), times the key's factor
    // 2^7 V scale / vs_ref into P (FP16, RNE); the row's sum takes each rounded P times the
    // factor's reciprocal (a mixed FP16 x FP32 FMA).
    // Elements are packed in pairs as the odd one completes (the product of the even one waits in
    // `prv`), and the pair goes to its P register at once.
    typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
    auto exp_elem = [&](int rb, int v, float e, const float4 &rw, uint32_t (&pw)[2][8], float (&lsum)[2],
                        float (&prv)[2]) __attribute__((always_inline)) {
        const float prod = e * ((v & 1) ? rw.z : rw.x);
        uint32_t d;
        if (v & 1) {
            const half2_t h = {(_Float16)prv[rb], (_Float16)prod};
            d = __builtin_bit_cast(uint32_t, h);
            // the sum takes the packed halves themselves (mixed FMAs on the P register), so that it
            // sees exactly the operands the MFMA multiplies
            asm("v_fma_mix_f32 %0, %1, %2, %0 op_sel_hi:[1,0,0]" : "+v"(lsum[rb]) : "v"(d), "v"(rw.y));
            asm("v_fma_mix_f32 %0, %1, %2, %0 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "+v"(lsum[rb]) : "v"(d), "v"(rw.w));
            pw[rb][v >> 1] = d;
        } else {
            prv[rb] = prod;
            d = __builtin_bit_cast(uint32_t, prod);
        }
        return d;
    };

    // The first LDS reads of each phase are issued one phase early (prefetch_a at the end of phase
    // B, prefetch_b before the barrier), so that their latency overlaps the previous phase's tail
    // and the barrier. Both read buffers no phase writes until after the next barrier: K(n) was
    // staged in phase B of tile n - 2, V(n - 1) and the scales of tiles n - 1 and n earlier still.
    // (INT8 only: the FP16 staging keeps more registers live, and the early reads then spill)
    constexpr bool kEarly = kInt8;
    static_assert(kW64QRegs >= 3, "the first three QK steps take their Q^T chunks from registers");
    // (ko, vo: the K tile phase A reads and the V tile whose scales its products take)
    auto prefetch_a = [&](uint32_t ko, uint32_t vo, float4 &r0, half8 (&kop)[3]) __attribute__((always_inline)) {
        r0 = load_rv(vo, 0);
        const _Float16 *kr = ktile(ko).k + qk_key_row(i) * kKStride + 8 * kk;
#pragma unroll
        for (int c = 0; c < 3; c++) kop[c] = *reinterpret_cast<const half8 *>(kr + 16 * c);
    };
    const int vsw = (i >> 2) & 3;   // V^T rows 32dt + i share the swizzle of row i
    // V(n - 1)^T operand of PV step j (16-key step j / 8, dimension tile j % 8)
    auto vop = [&](int j) __attribute__((always_inline)) {
        const _Float16 *vt = vtile(vm1).v + i * kW64Keys;
        return *reinterpret_cast<const half8 *>(vt + 32 * (j & 7) * kW64Keys + 8 * ((2 * (j >> 3) + kk) ^ vsw));
    };
    auto prefetch_b = [&](float4 (&k4)[4], half8 (&vr)[kW64VAhead]) __attribute__((always_inline)) {
        load_scales(vc0, k4);
#pragma unroll
        for (int j = 0; j < kW64VAhead; j++) vr[j] = vop(j);
    };

    // Phase A of tile n: S(n) for both row blocks (K operands read three steps ahead) and the
    // exponentials of tile n - 1 (P(n - 1) and l), spread between the MFMAs. One path for every
    // n: after the last tile (n = ntiles) the MFMAs multiply the finite codes staged for keys past
    // the split, an S that phase B replaces with -inf. r0 (the probability factors of tile n - 1's
    // first key pair and their reciprocals) and the first three K operands come from prefetch_a.
    auto phase_a = [&](int n, floatx16 (&sc)[2], floatx16 (&sp)[2], const float (&dec)[2], half8 (&pn)[2][2],
                       const float4 &r0pre, const half8 (&kpre_in)[3], Raw &raw) __attribute__((always_inline)) {
        // INT8: V(n + 1) from the codes in raw, a half-word per step in the gaps of row block 0
        // (piece 4 + c / 4: word (c / 2) % 2, low or high halves by c % 2), then its codes reloaded
        // for tile n + 2
        W64VTile &vnext = vtile(vc1);
        uint32_t vw[2] = {0u, 0u};
        uint4 vh = make_uint4(0u, 0u, 0u, 0u);
        float4 r0own;
        half8 kown[3];
        if constexpr (!kEarly) prefetch_a(kcur, vm1, r0own, kown);
        // the probability factors of tile n - 1 and their reciprocals, a key pair per read, each
        // read two steps before its use
        float4 rq[2];
        rq[0] = kEarly ? r0pre : r0own;
        const half8 (&kpre)[3] = kEarly ? kpre_in : kown;
        float lsum[2] = {0.0f, 0.0f};
        // INT8: exp2 runs one step ahead of its use: the wave issues in order, and a product
        // right behind its exponential would stall for the transcendental's latency (FP16 KV:
        // in place, its larger staging registers leave no room for the two in flight)
        constexpr bool kAhead = kInt8;
        float ex[2] = {0.0f, 0.0f}, prv[2] = {0.0f, 0.0f};
        // P(n - 1) as it is packed, in fresh registers (inserting into the previous tile's P would
        // keep its registers live into this phase)
        uint32_t pw[2][8];
        if constexpr (kAhead) {
            ex[0] = __builtin_amdgcn_exp2f(sp[0][0]);
            ex[1] = __builtin_amdgcn_exp2f(sp[1][0]);
        }
        {
            const _Float16 *kr = ktile(kcur).k + qk_key_row(i) * kKStride + 8 * kk;
            half8 kop[4];                                       // K operands, read three steps ahead
            half8 qop_l[3][2];                                  // Q^T chunks from LDS, two steps ahead
#pragma unroll
            for (int c = 0; c < 3; c++) kop[c] = kpre[c];
#pragma unroll
            for (int c = 0; c < 16; c++) {
                if (c + 3 < 16) kop[(c + 3) & 3] = *reinterpret_cast<const half8 *>(kr + 16 * (c + 3));
                if ((c & 1) == 0 && c < 14) rq[((c >> 1) + 1) & 1] = load_rv(vm1, c + 2);
                if (c + 2 < 16 && c + 2 >= kW64QRegs)
#pragma unroll
                    for (int rb = 0; rb < 2; rb++) qop_l[(c + 2) % 3][rb] = qop_at(rb, c + 2);
                const half8 q0 = c < kW64QRegs ? qop[0][c < kW64QRegs ? c : 0] : qop_l[c % 3][0];
                const half8 q1 = c < kW64QRegs ? qop[1][c < kW64QRegs ? c : 0] : qop_l[c % 3][1];
                // each step's vector work lies between its MFMA (after_mfma on its inputs) and the
                // next one (before_mfma on its results)
                auto gap = [&](int rb) __attribute__((always_inline)) {
                    const int cz = kAhead ? (c < 15 ? c + 1 : 15) : c;
                    float z = sp[rb][cz];
                    after_mfma(z, lsum[rb]);
                    sp[rb][cz] = z;
                    float e;
                    if constexpr (kAhead) {
                        e = ex[rb];
                        if (c < 15) ex[rb] = __builtin_amdgcn_exp2f(z);
                    } else {
                        e = __builtin_amdgcn_exp2f(z);
                    }
                    const uint32_t d = exp_elem(rb, c, e, rq[(c >> 1) & 1], pw, lsum, prv);
                    before_mfma(lsum[rb], ex[rb], d);
                };
                if (c == 0)
                    s_mfma_first(sc[0], kop[c & 3], q0);
                else
                    s_mfma(sc[0], kop[c & 3], q0);
                gap(0);
                if constexpr (kVinA) {
                    const int piece = 4 + c / 4, sub = c & 3;
                    if (sub == 0) {
                        uint32_t x[4];
                        piece_words(raw, piece, x);
                        vw[0] = x[0];
                        vw[1] = x[1];
                    }
                    if (sub == 0) i8x4_to_f16_sdwa_lo(vw[0], vh.x, vh.y);
                    if (sub == 1) i8x4_to_f16_sdwa_hi(vw[0], vh.x, vh.y);
                    if (sub == 2) i8x4_to_f16_sdwa_lo(vw[1], vh.z, vh.w);
                    if (sub == 3) {
                        i8x4_to_f16_sdwa_hi(vw[1], vh.z, vh.w);
                        store_piece(kbuf[0], vnext, piece, vh);   // (a V piece: the K tile is not touched)
                    }
                }
                if (c == 0)
                    s_mfma_first(sc[1], kop[c & 3], q1);
                else if (c < 15)
                    s_mfma(sc[1], kop[c & 3], q1);
                else
                    s_mfma_last(sc[1], kop[c & 3], q1);
                gap(1);
            }
        }
        if constexpr (kVinA) load_part(raw, min(kbeg + (uint32_t)(n + 2) * kW64Keys, last_key0), 2);
#pragma unroll
        for (int rb = 0; rb < 2; rb++) {
#pragma unroll
            for (int u = 0; u < 2; u++)
                pn[rb][u] = __builtin_bit_cast(half8, make_uint4(pw[rb][4 * u], pw[rb][4 * u + 1], pw[rb][4 * u + 2], pw[rb][4 * u + 3]));
            l[rb] = fmaf(l[rb], dec[rb], lsum[rb]);
            // P(n - 1) complete here, before the barrier: phase B's assembly MFMAs read it, and
            // the compiler pads no wait states for them
            asm volatile("" : "+v"(pn[rb][0]), "+v"(pn[rb][1]));
        }
    };

    auto row_max = [&](const floatx16 &s) __attribute__((always_inline)) {
        const float ma = max3f(s[0], s[1], s[2]), mb = max3f(s[3], s[4], s[5]), mc = max3f(s[6], s[7], s[8]);
        const float md = max3f(s[9], s[10], s[11]), me = max3f(s[12], s[13], s[14]);
        return pair_max(max3f(max3f(ma, mb, mc), max3f(md, me, s[15]), s[15]));
    };

    // Phase B of tile n: O += V(n - 1)^T P(n - 1) (V operands read kW64VAhead steps ahead),
    // interleaved with S(n)'s scaling (K scale, log2(e) / 16, less the running maximum) and its row
    // maxima. `need` reports the rows whose maximum grows by more than 2^15 (or that meet their
    // first key): fix_softmax handles those and the causal mask. One code path for every tile (the
    // accumulators must not meet branches): before the first tile P is zero and the V buffer it
    // reads is zero-filled; after the last (past), S is -inf, which leaves m, l and P unchanged.
    auto phase_b = [&](int n, floatx16 (&sc)[2], const half8 (&pp)[2][2], bool (&need)[2], float (&ymax)[2], bool past,
                       Raw &raw, const float4 (&k4pre)[4], const half8 (&vpre_in)[kW64VAhead], float4 &r4n,
                       half8 (&kopn)[3]) __attribute__((always_inline)) {
        float4 k4own[4];
        half8 vown[kW64VAhead];
        if constexpr (!kEarly) prefetch_b(k4own, vown);
        const float4 (&k4)[4] = kEarly ? k4pre : k4own;
        const half8 (&vpre)[kW64VAhead] = kEarly ? vpre_in : vown;
        const uint32_t key2 = kbeg + (uint32_t)(n + 2) * kW64Keys;
        W64KTile &kdst = ktile(kcur);   // tile n's, read in phase A of tile n
        W64VTile &vdst = vtile(vc2);    // tile n - 2's, read in phase B of tile n - 1
        float add[2];
        float mq[2] = {m[0], m[1]};
        asm volatile("" : "+v"(mq[0]), "+v"(mq[1]));   // computed in this phase, not hoisted into phase A
#pragma unroll
        for (int rb = 0; rb < 2; rb++)   // past the last tile: -inf for every key, whatever the (finite) S and K scales
            add[rb] = past ? -INFINITY : -(mq[rb] == -INFINITY ? 0.0f : mq[rb]);
        // step j < 8 scales elements 2j, 2j + 1 of each row block; steps 8-9 take the maxima
        auto scale_pair = [&](int rb, int j) __attribute__((always_inline)) {
            // in place, held before the next MFMA (a tie on copies of the inputs would add moves)
            const float4 &kq = k4[j >> 1];
            sc[rb][2 * j] = fmaf(sc[rb][2 * j], (j & 1) ? kq.z : kq.x, add[rb]);
            sc[rb][2 * j + 1] = fmaf(sc[rb][2 * j + 1], (j & 1) ? kq.w : kq.y, add[rb]);
            before_mfma(sc[rb][2 * j], sc[rb][2 * j + 1]);
        };
        float mpart[2][2];
        auto max_piece = [&](int rb, int j) __attribute__((always_inline)) {
            const floatx16 &t = sc[rb];
            if (j == 8) {
                mpart[rb][0] = max3f(max3f(t[0], t[1], t[2]), max3f(t[3], t[4], t[5]), max3f(t[6], t[7], t[8]));
                mpart[rb][1] = max3f(max3f(t[9], t[10], t[11]), max3f(t[12], t[13], t[14]), t[15]);
                before_mfma(mpart[rb][0], mpart[rb][1]);
            } else if (j == 9) {
                ymax[rb] = pair_max(max3f(mpart[rb][0], mpart[rb][1], mpart[rb][1]));
                need[rb] = ymax[rb] > thr[rb];   // > kRebase, or a row's first keys (thr = -inf while m is)
            }
        };
        uint32_t xs[4], key3 = 0;
        uint4 hs;
        half8 vring[kW64VAhead + 1];
#pragma unroll
        for (int j = 0; j < kW64VAhead; j++) vring[j] = vpre[j];
#pragma unroll
        for (int j = 0; j < 16; j++) {
            if (j + kW64VAhead < 16) vring[(j + kW64VAhead) % (kW64VAhead + 1)] = vop(j + kW64VAhead);
            const half8 va = vring[j % (kW64VAhead + 1)];
            // Work per gap (about seven instructions beside each MFMA): steps 0-7 scale two S
            // elements per row block; step 3 stages the scales of tile n + 2, and its pieces follow
            // (INT8: the K pieces 0-3 at steps 4, 6, 8, 10, one word of codes per gap — its V is
            // staged in phase A; FP16: pieces j - 4 at steps 4-11); the loads of tile n + 3 follow
            // as their registers free up (scales at step 4, K codes after the last K piece, FP16 V
            // codes at 12), about a tile before their use; steps 12-13 take the maxima; step 14
            // issues phase A's first reads of tile n + 1.
            const bool kstep = kInt8 && j >= 4 && j < 12 && (j & 1) == 0;
            const int kpiece = (j - 4) >> 1;
            o_mfma(o[0][j & 7], va, pp[0][j >> 3]);
            if (j < 8) scale_pair(0, j);
            if (j >= 12) max_piece(0, j - 4);
            if (kstep) {   // (the conversion is volatile assembly: it stays in this gap)
                piece_words(raw, kpiece, xs);
                i8x4_to_f16_sdwa(xs[0], hs.x, hs.y);
            }
            if (!kInt8 && j >= 4 && j < 12) {   // FP16: the whole piece (copies and V^T transposes)
                uint32_t x[4];
                piece_words(raw, j - 4, x);
                after_mfma(x[0], x[1], x[2], x[3]);
                stage_piece(kdst, vdst, j - 4, x);
            }
            if (j == 3) stage_scales(vdst, key2, raw);
            if (j == (kVinA ? 12 : 8)) load_part(raw, key3, 1);   // K codes of tile n + 3
            if (!kVinA && j == 12) load_part(raw, key3, 2);        // V codes of tile n + 3
            o_mfma(o[1][j & 7], va, pp[1][j >> 3]);
            if (j < 8) scale_pair(1, j);
            if (j >= 12) max_piece(1, j - 4);
            if (kstep) {
                i8x4_to_f16_sdwa(xs[1], hs.z, hs.w);
                store_piece(kdst, vdst, kpiece, hs);
            }
            if (j == 4) {
                key3 = min(key2 + kW64Keys, last_key0);   // once per tile; its arithmetic stays here
                asm volatile("" : "+s"(key3));
                load_part(raw, key3, 0);   // scales of tile n + 3
            }
            if (kEarly && j == 14) prefetch_a(kcur ^ kKT, vc0, r4n, kopn);   // after the last tile: unused reads
        }
    };

    // The general case of tile n, after phase B: the causal mask, the lazy running maximum (a row
    // rebases only when its maximum grows by more than 2^kRebase, so exponentials stay <= 2^15 and
    // P in FP16 range; a rebase rescales O, so rarer ones save most of that work): S is
    // shifted by the rebase, `dec` is the factor l takes before tile n's sum joins it.
    // `rescale_row` reports the rows whose O must take dec: a rebase of a row that had keys before.
    // A row's first rebase finds O zero; any other takes dec, also where exp2(-ymax) underflows to 0
    // (a maximum that grows by more than 2^149 leaves nothing of the earlier keys).
    auto fix_softmax = [&](int n, floatx16 (&sc)[2], float (&ymax)[2], float (&dec)[2], bool (&rescale_row)[2],
                           bool masked) __attribute__((always_inline)) {
        const uint32_t key0 = kbeg + (uint32_t)n * kW64Keys;
        if (masked) {
#pragma unroll
            for (int rb = 0; rb < 2; rb++) {
#pragma unroll
                for (int v = 0; v < 16; v++)
                    if (key0 + 16 * (v >> 3) + 8 * kk + (v & 7) > limit[rb]) sc[rb][v] = -INFINITY;
                ymax[rb] = row_max(sc[rb]);
            }
        }
#pragma unroll
        for (int rb = 0; rb < 2; rb++) {
            const bool rebase = ymax[rb] > kRebase || (m[rb] == -INFINITY && ymax[rb] > -INFINITY);
            const float mref = m[rb] == -INFINITY ? 0.0f : m[rb];
            dec[rb] = rebase ? (m[rb] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(-ymax[rb])) : 1.0f;
            rescale_row[rb] = rebase && m[rb] != -INFINITY;
            m[rb] = rebase ? mref + ymax[rb] : m[rb];
            thr[rb] = m[rb] == -INFINITY ? -INFINITY : kRebase;
            if (rebase) {
#pragma unroll
                for (int v = 0; v < 16; v++) sc[rb][v] = sc[rb][v] - ymax[rb];
            }
        }
    };

    // In place in the accumulator registers: written as arithmetic, a rescale inside a branch
    // moves the accumulators out of them. The no-ops cover the wait states between the last MFMA
    // or VALU write and the accumulator reads and writes.
    auto rescale = [&](const float (&decay)[2]) __attribute__((always_inline)) {
        asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7");
#pragma unroll
        for (int rb = 0; rb < 2; rb++)
#pragma unroll
            for (int dt = 0; dt < 8; dt++)
#pragma unroll
                for (int e = 0; e < 16; e++) {
                    float t;
                    asm volatile(
                        "v_accvgpr_read_b32 %1, %0\n\ts_nop 1\n\tv_mul_f32 %1, %1, %2\n\ts_nop 1\n\t"
                        "v_accvgpr_write_b32 %0, %1"
                        : "+a"(o[rb][dt][e]), "=&v"(t)
                        : "v"(decay[rb]));
                }
        asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7");
    };

    // S(n - 1), scaled and shifted (exp2 of it is P(n - 1) before the V scales), and the factor
    // l takes before its sum joins: tile -1 has no keys
    floatx16 sp[2];
    float dec[2] = {1.0f, 1.0f};
#pragma unroll
    for (int rb = 0; rb < 2; rb++)
#pragma unroll
        for (int v = 0; v < 16; v++) sp[rb][v] = -INFINITY;
    float4 r4n;
    half8 kopn[3];
    if constexpr (kEarly) prefetch_a(kcur, vm1, r4n, kopn);
    for (int n = 0; n <= ntiles; n++) {
        // the accumulators live in the accumulator registers across iterations
#pragma unroll
        for (int rb = 0; rb < 2; rb++)
#pragma unroll
            for (int dt = 0; dt < 8; dt++) asm volatile("" : "+a"(o[rb][dt]));
        floatx16 sc[2];
        phase_a(n, sc, sp, dec, pb, r4n, kopn, raw);
        // The barrier between the phases, with phase B's first reads in flight across it: this
        // wave's LDS writes (the staging of phase B of tile n - 1) and phase A's reads are complete
        // first, as a work-group barrier's release would have them, and the assembly barrier keeps
        // the compiler from waiting for the reads issued after that.
        float4 k4[4];
        half8 vpre[kW64VAhead];
        if constexpr (kEarly) {
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            prefetch_b(k4, vpre);
            asm volatile("s_barrier" ::: "memory");
            // odd waves start phase B half an MFMA step later: the waves run in step after the
            // barrier, and an LDS write holds its wave until the LDS has taken it, so staging
            // writes issued by all four at once wait on each other (measured 1.9% per tile)
            if (wave & 1) asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7");
        } else {
            __syncthreads();
        }
        bool need[2];
        float ymax[2];
        phase_b(n, sc, pb, need, ymax, n == ntiles, raw, k4, vpre, r4n, kopn);
        dec[0] = dec[1] = 1.0f;
        const bool masked = kbeg + (uint32_t)n * kW64Keys + kW64Keys - 1 > wave_min_limit;
        if (masked | ((__ballot(need[0]) | __ballot(need[1])) != 0)) {   // bitwise: both sides computed
            bool rescale_row[2];
            fix_softmax(n, sc, ymax, dec, rescale_row, masked);
            // a rebase scales what O holds (through tile n - 1) before P(n) joins it (rows that do
            // not rebase take dec = 1; a first rebase, dec = 0, finds O zero)
            if (__ballot(rescale_row[0] | rescale_row[1])) rescale(dec);
        }
#pragma unroll
        for (int rb = 0; rb < 2; rb++) sp[rb] = sc[rb];
        kcur ^= kKT;
        const uint32_t t = vm1;
        vm1 = vc0;
        vc0 = vc1;
        vc1 = vc2;
        vc2 = t;
    }
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7");   // the last MFMAs' results, before O is read
#pragma unroll
    for (int rb = 0; rb < 2; rb++) l[rb] += __shfl_xor(l[rb], 32, 64);   // the two lanes of a row summed disjoint keys

    // ---- epilogue: lane (i, kk) holds O^T[d][row] for d = 32dt + 8(v/4) + 4kk + v%4. O sums the
    // operands 2^7 e vs / vs_ref times the codes, so vs_ref / 2^7 turns O / l into values.
    const float vs_out = vs_ref * (1.0f / kPScale);
    if (p.splits == 1) {
        // The row's 32 gate loads go out together before its first store: y may alias the query
        // buffer, and the compiler, unable to tell y from the gate, would otherwise hold each load
        // behind the previous store (one memory round trip per 16 bytes of output).
#pragma unroll
        for (int rb = 0; rb < 2; rb++) {
            const uint32_t token = my_row[rb] / 8, head = g * 8 + my_row[rb] % 8;
            const size_t base = ((size_t)token * 16 + head) * 256;
            const float inv = vs_out / l[rb];
            float4 gv[32];
#pragma unroll
            for (int c = 0; c < 32; c++)
                gv[c] = row_valid[rb] ? *reinterpret_cast<const float4 *>(p.gate + base + 32 * (c >> 2) + 8 * (c & 3) + 4 * kk)
                                      : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            if (!row_valid[rb]) continue;
#pragma unroll
            for (int dt = 0; dt < 8; dt++)
#pragma unroll
                for (int vq = 0; vq < 4; vq++) {
                    const int d = 32 * dt + 8 * vq + 4 * kk;
                    const float4 g4 = gv[4 * dt + vq];
                    float4 out;
                    out.x = o[rb][dt][4 * vq + 0] * inv * sigmoidf(g4.x);
                    out.y = o[rb][dt][4 * vq + 1] * inv * sigmoidf(g4.y);
                    out.z = o[rb][dt][4 * vq + 2] * inv * sigmoidf(g4.z);
                    out.w = o[rb][dt][4 * vq + 3] * inv * sigmoidf(g4.w);
                    *reinterpret_cast<float4 *>(p.y + base + d) = out;
                }
        }
        return;
    }
    // Split partials: O^T / l per row, through LDS so that every store instruction writes 1 KB
    // of whole rows (16-byte pieces of 32 rows each reach HBM as partial lines). A row is written
    // as FP16 when its largest |O^T / l| x vs_ref / 2^7 (an output magnitude) is at most
    // kNarrowPartial, where FP16's relative 2^-12 keeps the error under 1e-3; otherwise as FP32
    // (heavy-tailed V reaches |y| ~ 16: FP16 there is 4e-3 off, and no 16-bit format meets both
    // the 2e-3 bar and the reference's per-element bound for every value of such a row). Each row
    // has a 1 KB slot; FP16 rows fill its first half. Wave w stages rows (16-byte chunks
    // XOR-swizzled by row) in a 32 KB region no other wave uses: K tiles, V tiles 0-1, V tiles
    // 2-3, the Q^T chunks; FP32 rows in two passes of 32.
    static_assert(sizeof(kbuf) >= 32768 && 2 * sizeof(W64VTile) >= 32768 && sizeof(qlds) >= 32768,
                  "an LDS region per wave holds 32 KB of rows");
    __syncthreads();   // every wave has read its last tile
    unsigned char *ostage = wave == 0   ? reinterpret_cast<unsigned char *>(kbuf)
                            : wave == 1 ? reinterpret_cast<unsigned char *>(&vbuf[0])
                            : wave == 2 ? reinterpret_cast<unsigned char *>(&vbuf[2])
                                        : reinterpret_cast<unsigned char *>(qlds);
    unsigned char *pbase = reinterpret_cast<unsigned char *>(p.partial) +
                           (((size_t)g * p.tiles + tile) * p.splits + split) * kPartialBytes;
    // Every row is staged as FP16 first, each row's largest magnitude taken on the way; the rows
    // whose outputs are too large are then staged again as FP32 from the accumulators (chosen per
    // row: with one choice per wave, a single element above the bound among a wave's 16K sent all
    // 64 rows to FP32, 5 MB per 512-row chunk on the bench's data)
    typedef _Float16 half4 __attribute__((ext_vector_type(4)));
    float inv_l[2], zmax[2] = {0.0f, 0.0f};
#pragma unroll
    for (int rb = 0; rb < 2; rb++) {
        const int row = 32 * rb + i;   // of the wave's 64
        inv_l[rb] = l[rb] > 0.0f ? 1.0f / l[rb] : 0.0f;
#pragma unroll
        for (int dt = 0; dt < 8; dt++)
#pragma unroll
            for (int vq = 0; vq < 4; vq++) {
                const int chunk = 4 * dt + vq;   // dimensions 8 chunk .. 8 chunk + 7; this lane's half at 4 kk
                const float z0 = o[rb][dt][4 * vq] * inv_l[rb], z1 = o[rb][dt][4 * vq + 1] * inv_l[rb];
                const float z2 = o[rb][dt][4 * vq + 2] * inv_l[rb], z3 = o[rb][dt][4 * vq + 3] * inv_l[rb];
                zmax[rb] = max3f(zmax[rb], max3f(fabsf(z0), fabsf(z1), fabsf(z2)), fabsf(z3));
                const half4 hv = {(_Float16)z0, (_Float16)z1, (_Float16)z2, (_Float16)z3};
                *reinterpret_cast<half4 *>(ostage + row * 512 + ((chunk ^ (row & 31)) * 16) + 8 * kk) = hv;
            }
    }
    // wide[rb]: bit i set when row 32 rb + i of the wave needs FP32 (lanes i and i + 32 hold its two
    // halves of the dimensions)
    uint32_t wide[2];
#pragma unroll
    for (int rb = 0; rb < 2; rb++) {
        const float z = fmaxf(zmax[rb], __shfl_xor(zmax[rb], 32, 64));
        wide[rb] = (uint32_t)__ballot(z * vs_out > kNarrowPartial);
    }
    if (kk == 0) {
#pragma unroll
        for (int rb = 0; rb < 2; rb++) {
            const int local_row = 64 * wave + 32 * rb + i;
            float *stat = reinterpret_cast<float *>(pbase + 2 * kPartialRegion);
            stat[local_row] = m[rb];
            stat[kTileRows + local_row] = l[rb];
            stat[2 * kTileRows + local_row] = (wide[rb] >> i) & 1u ? -vs_out : vs_out;   // the sign carries the format
        }
    }
    unsigned char *pw = pbase + (size_t)(64 * wave) * 512;   // the wave's rows are contiguous
    if ((wide[0] | wide[1]) == 0u) {
#pragma unroll
        for (int it = 0; it < 32; it++) {
            const int row = 2 * it + (lane >> 5), chunk = lane & 31;
            const uint4 v = *reinterpret_cast<const uint4 *>(ostage + row * 512 + ((chunk ^ (row & 31)) * 16));
            *reinterpret_cast<uint4 *>(pw + (size_t)it * 1024 + lane * 16) = v;
        }
        return;
    }
    // some rows FP32: the FP16 rows first (iteration it stores rows 2 it and 2 it + 1, a half-wave
    // each), then the FP32 rows of each row block that has any
#pragma unroll
    for (int it = 0; it < 32; it++) {
        const int row = 2 * it + (lane >> 5), chunk = lane & 31;
        if ((wide[it >> 4] >> (row & 31)) & 1u) continue;
        const uint4 v = *reinterpret_cast<const uint4 *>(ostage + row * 512 + ((chunk ^ (row & 31)) * 16));
        *reinterpret_cast<uint4 *>(pw + (size_t)it * 1024 + lane * 16) = v;
    }
    // (the accumulators are read by explicit moves, so that the compiler holds no vector-register
    // copies of them from the FP16 staging across the branch)
    auto acc_read = [&](const float &a) __attribute__((always_inline)) {
        float t;
        asm volatile("v_accvgpr_read_b32 %0, %1" : "=v"(t) : "a"(a));
        return t;
    };
#pragma unroll
    for (int rb = 0; rb < 2; rb++) {
        if (wide[rb] == 0u) continue;   // wave-uniform
#pragma unroll
        for (int dt = 0; dt < 8; dt++)
#pragma unroll
            for (int vq = 0; vq < 4; vq++) {
                const int chunk = 8 * dt + 2 * vq + kk;   // dimensions 4 chunk .. 4 chunk + 3
                const float4 fv = make_float4(
                    acc_read(o[rb][dt][4 * vq]) * inv_l[rb], acc_read(o[rb][dt][4 * vq + 1]) * inv_l[rb],
                    acc_read(o[rb][dt][4 * vq + 2]) * inv_l[rb], acc_read(o[rb][dt][4 * vq + 3]) * inv_l[rb]);
                *reinterpret_cast<float4 *>(ostage + i * 1024 + ((chunk ^ i) * 16)) = fv;
            }
#pragma unroll
        for (int r = 0; r < 32; r++) {   // lanes 0-31: dimensions 0-127 to region A, lanes 32-63 to B
            if (((wide[rb] >> r) & 1u) == 0u) continue;   // wave-uniform
            const uint4 v = *reinterpret_cast<const uint4 *>(ostage + r * 1024 + ((lane ^ r) * 16));
            *reinterpret_cast<uint4 *>(pw + (lane >> 5) * kPartialRegion + (size_t)(32 * rb + r) * 512 + (lane & 31) * 16) = v;
        }
    }
}

// Merges the split partials of prefill_w64_kernel (O^T / l, FP16 or FP32 per the row's format,
// then m, l, +-vs_ref / 2^7): one wave per logical row, four dimensions per lane, eight splits per
// step with a running maximum. The FP16 loads go out with the statistics; a split whose rows are
// FP32 is read again in full once its format is known.
__global__ __launch_bounds__(256) void prefill_combine_kernel(PrefillParams p) {
    const uint32_t lane = threadIdx.x & 63;
    uint32_t bx = blockIdx.x, tile = blockIdx.y, g = blockIdx.z;
    if (p.remap == 2) {   // the XCD whose work-groups wrote the tile's partials (still in its L2)
        const uint32_t xcd = bx % 8, idx = bx / 8, pair = xcd + 8 * (idx / (kTileRows / 4));
        bx = idx % (kTileRows / 4);
        g = pair % 2;
        tile = pair / 2;
    }
    const uint32_t local_row = bx * 4 + (threadIdx.x >> 6);
    const uint32_t row = tile * kTileRows + local_row;
    if (row >= p.rows * 8) return;   // wave-uniform
    const unsigned char *base = reinterpret_cast<const unsigned char *>(p.partial) +
                                ((size_t)g * p.tiles + tile) * p.splits * kPartialBytes;
    const uint32_t token = row / 8, head = g * 8 + row % 8;
    const size_t at = ((size_t)token * 16 + head) * 256 + 4 * lane;
    const float4 gv = *reinterpret_cast<const float4 *>(p.gate + at);
    typedef _Float16 half4 __attribute__((ext_vector_type(4)));
    float mrun = -INFINITY, lsum = 0.0f;
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (uint32_t s0 = 0; s0 < p.splits; s0 += 8) {
        float ms[8], ls[8], ws[8];
        half4 hs[8];
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const uint32_t s = min(s0 + j, p.splits - 1);
            const unsigned char *part = base + s * kPartialBytes;
            const float *stat = reinterpret_cast<const float *>(part + 2 * kPartialRegion);
            ms[j] = s0 + j < p.splits ? stat[local_row] : -INFINITY;
            ls[j] = stat[kTileRows + local_row];
            ws[j] = stat[2 * kTileRows + local_row];
            hs[j] = *reinterpret_cast<const half4 *>(part + (size_t)local_row * 512 + 8 * lane);
        }
        float4 os[8];
        bool wide = false;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            os[j] = make_float4((float)hs[j].x, (float)hs[j].y, (float)hs[j].z, (float)hs[j].w);
            wide |= ws[j] < 0.0f;
        }
        if (wide) {   // wave-uniform and rare: some split's rows are FP32
#pragma unroll
            for (int j = 0; j < 8; j++)
                if (ws[j] < 0.0f) {
                    const uint32_t s = min(s0 + j, p.splits - 1);
                    os[j] = *reinterpret_cast<const float4 *>(base + s * kPartialBytes + (lane >> 5) * kPartialRegion +
                                                              (size_t)local_row * 512 + 16 * (lane & 31));
                }
        }
        float mstep = ms[0];
#pragma unroll
        for (int j = 1; j < 8; j++) mstep = fmaxf(mstep, ms[j]);
        if (mstep == -INFINITY) continue;   // wave-uniform: every split of the step is empty
        const float mnew = fmaxf(mrun, mstep);
        const float decay = mrun == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mrun - mnew);
        mrun = mnew;
        lsum *= decay;
        acc.x *= decay;
        acc.y *= decay;
        acc.z *= decay;
        acc.w *= decay;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            if (ms[j] == -INFINITY) continue;
            const float f = __builtin_amdgcn_exp2f(ms[j] - mnew);
            const float lf = ls[j] * f;
            const float wf = lf * fabsf(ws[j]);
            lsum += lf;
            acc.x += os[j].x * wf;
            acc.y += os[j].y * wf;
            acc.z += os[j].z * wf;
            acc.w += os[j].w * wf;
        }
    }
    const float inv = 1.0f / lsum;
    float4 out;
    out.x = acc.x * inv * sigmoidf(gv.x);
    out.y = acc.y * inv * sigmoidf(gv.y);
    out.z = acc.z * inv * sigmoidf(gv.z);
    out.w = acc.w * inv * sigmoidf(gv.w);
    *reinterpret_cast<float4 *>(p.y + at) = out;
}

inline bool aligned(const void *ptr, uintptr_t a) { return (reinterpret_cast<uintptr_t>(ptr) & (a - 1)) == 0; }

}  // namespace

namespace {

const char *launch_prefill(Context &c, const View *b, const boot_kernel_args &a, bool int8) {
    const uint64_t rows = a.m;
    if (rows == 0) return nullptr;
    BOOT_REQUIRE(a.a == 8 || a.a == 0, "online attention groups 8 query heads per KV head (A = 8)");
    BOOT_REQUIRE((uint64_t)a.k == (uint64_t)a.pos + rows, "K must equal Position + M");
    const uint64_t keys = a.k;
    BOOT_REQUIRE(keys <= 262144, "attended length exceeds the 262144-token window");
    BOOT_REQUIRE(b[0].bytes >= rows * 8192, "packed FP16 query smaller than rows*4096 halves");
    if (int8) {
        BOOT_REQUIRE(b[1].bytes >= keys * 512, "K cache smaller than K tokens");
        BOOT_REQUIRE(b[2].bytes >= value_bytes(keys), "V cache smaller than whole pages of K tokens");
        BOOT_REQUIRE(b[5].bytes >= keys * 8 && b[6].bytes >= keys * 8, "KV scale buffers smaller than K tokens");
        BOOT_REQUIRE(aligned(b[5].ptr, 4) && aligned(b[6].ptr, 4), "scale bindings misaligned");
    } else {
        BOOT_REQUIRE(b[1].bytes >= keys * 1024 && b[2].bytes >= keys * 1024, "FP16 K/V cache smaller than K tokens");
    }
    BOOT_REQUIRE(b[3].bytes >= rows * 16384 && b[4].bytes >= rows * 16384, "gate/output smaller than rows*4096 floats");
    BOOT_REQUIRE(aligned(b[0].ptr, 16) && aligned(b[1].ptr, 16) && aligned(b[2].ptr, 16) && aligned(b[3].ptr, 16) &&
                     aligned(b[4].ptr, 16),
                 "bindings misaligned (q, k, v, gate, y need 16 bytes)");
    // Chunks of at most 64 rows whose rows x keys stay within kDecodeRouteWork go to the decode
    // kernel (one work-group per row, KV group and split of the keys): at (0, 33) 7.6 against
    // 25.4 us, at (2048, 33) 24.8 against 38.4 us; each row reads the keys again, so at (8192, 33)
    // it would take 81 against 44 us.
    if (int8 && rows <= 64 && rows * keys <= kDecodeRouteWork) return launch_online_int8_as_decode(c, b, a);
    PrefillParams p;
    p.q = (const _Float16 *)b[0].ptr;
    p.k = b[1].ptr;
    p.v = b[2].ptr;
    p.gate = (const float *)b[3].ptr;
    p.y = (float *)b[4].ptr;
    p.ks = int8 ? (const float *)b[5].ptr : nullptr;
    p.vs = int8 ? (const float *)b[6].ptr : nullptr;
    p.rows = (uint32_t)rows;
    p.pos = a.pos;
    p.keys = (uint32_t)keys;
    // 256-row work-groups of 4 waves (one per SIMD), one per CU, for both storage formats: the
    // FP16-KV control runs the same schedule with FP16 staging, so that the two differ only in
    // the cache they read.
    p.tiles = (uint32_t)((rows * 8 + kTileRows - 1) / kTileRows);
    // split-K: enough blocks to fill the CUs, each split at least 256 keys
    const uint64_t base_blocks = 2ull * p.tiles;
    const uint64_t want = (uint64_t)std::max(1, context_cus(c));
    uint64_t splits = std::max<uint64_t>(1, (want + base_blocks - 1) / base_blocks);
    splits = std::min<uint64_t>(splits, std::max<uint64_t>(1, keys / 256));
    uint64_t split_keys = (keys + splits - 1) / splits;
    split_keys = (split_keys + kW64Keys - 1) / kW64Keys * kW64Keys;
    splits = (keys + split_keys - 1) / split_keys;
    p.splits = (uint32_t)splits;
    p.split_keys = (uint32_t)split_keys;
    const uint64_t blocks = base_blocks * splits;
    // Block placement (work-groups go to the XCDs round-robin by block index). With split-K and a
    // multiple of 8 (group, tile) pairs, all splits of a pair share one XCD: its 128 KB query tile is
    // read into one L2 instead of four (4 MB instead of 16 MB per 512-row chunk, in the launch's
    // opening burst), the combine finds the partials in that L2, and each K/V tile is read by four
    // XCDs during the key loop (attention +0.7%, combine -22%, step -0.5 to -0.9%, A/B on one box).
    // Otherwise the blocks of one key range share an XCD when the splits tile the XCDs evenly.
    p.remap = splits > 1 && (2 * p.tiles) % 8 == 0 ? 2u : ((2 * splits) % 8 == 0) ? 1u : 0u;
    p.partial = nullptr;
    if (splits > 1) {
        p.partial = (float *)context_workspace(c, base_blocks * splits * kPartialBytes);
        BOOT_REQUIRE(p.partial, "cannot allocate prefill split workspace");
    }
    if (int8)
        launch_timed(c, "prefill_w64_kernel", prefill_w64_kernel<true>, dim3((uint32_t)blocks), dim3(256), p);
    else
        launch_timed(c, "prefill_w64_fp16_kernel", prefill_w64_kernel<false>, dim3((uint32_t)blocks), dim3(256), p);
    if (splits > 1) {
        context_split(c, int8 ? "attention_online_int8.combine" : "attention_online_fp16.combine");
        const dim3 cgrid = p.remap == 2 ? dim3(kTileRows / 4 * p.tiles * 2) : dim3(kTileRows / 4, p.tiles, 2);
        launch_timed(c, "prefill_combine_kernel", prefill_combine_kernel, cgrid, dim3(256), p);
    }
    return nullptr;
}

}  // namespace

const char *launch_online_int8(Context &c, const View *b, int count, const boot_kernel_args &a, const uint32_t *) {
    // bindings (DeviceAttention.cs:69): q FP16 grouped, k, v, gate, y, ks, vs; M rows, K = pos + M,
    // Position = pos, A = 8 heads per group.
    BOOT_REQUIRE(count >= 7, "attention_online_int8 needs 7 bindings: q, k, v, gate, y, ks, vs");
    return launch_prefill(c, b, a, true);
}

const char *launch_online_fp16(Context &c, const View *b, int count, const boot_kernel_args &a, const uint32_t *) {
    // bindings (DeviceAttention.cs:62-63): q FP16 grouped, k FP16, v FP16 (token-major), gate, y
    BOOT_REQUIRE(count >= 5, "attention_online_q32_k256_s8_g8_r2 needs 5 bindings: q, k, v, gate, y");
    return launch_prefill(c, b, a, false);
}

}  // namespace boot
