// Shared types and helpers of the gfx950 ColabFold kernels: MFMA operand types, status
// reporting, buffer validation and the XCD-aware work-item mapping.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>

#include "colabfold_gfx950.h"

namespace clk {

// ---- device side --------------------------------------------------------------------------

typedef _Float16 half_t;
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef float float8v __attribute__((ext_vector_type(8)));

constexpr int kWave = 64;

// A masked key's logit, replacing its biased score (the reference's AlphaFold fp16 mask bias):
// -inf would leave inf - inf on a row whose keys are all masked (cuda/volta_attn.h:9-11).
constexpr float kMaskedLogit = -1.0e4f;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kMaskedLogit2 = kMaskedLogit * kLog2e;  // in the exp2 domain

// One v_mfma_f32_16x16x32_f16: D[16x16] += A[16x32] B[32x16], fp32 accumulate. Lane l supplies
// A row (l % 16) and B column (l % 16), eight contraction slots each (slot group l / 16), and
// holds D rows 4 (l / 16) .. +3 of column l % 16.
__device__ __forceinline__ float4v mfma16x16x32(half8 a, half8 b, float4v c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// s_waitcnt vmcnt(0) with the other counters left alone (gfx9 encoding: vmcnt in bits 3:0 and
// 15:14, expcnt 6:4, lgkmcnt 11:8), for __builtin_amdgcn_s_waitcnt: unlike an asm statement, the
// compiler's own wait insertion sees it and knows that no vector memory access is in flight after
// it.
constexpr int kWaitVm0 = 0x0F70;

// Activations of the fused ops are fp16 (the reference's F16 contract) or bf16 (BF). Loads keep
// the raw 16-bit patterns in half8 registers and convert where the value is used; a bf16 value
// converts to fp16 exactly within fp16's normal range, so MFMA operands stay fp16. Results are
// rounded to the activation type once, on store (v_cvt_pk_bf16_f32 for bf16).
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

template <bool BF>
__device__ __forceinline__ float act_get(half8 raw, int e) {
    if constexpr (BF) {
        return (float)__builtin_bit_cast(bf16x8, raw)[e];
    } else {
        return (float)raw[e];
    }
}

// v rounded to the activation type, as a raw 16-bit pattern
template <bool BF>
__device__ __forceinline__ half_t act_cvt(float v) {
    if constexpr (BF) {
        return __builtin_bit_cast(half_t, (__bf16)v);
    } else {
        return (half_t)v;
    }
}

// LDS row of tile row x, for operand tiles whose A row r of block b is
//   x = per (r / 4) + 4 b + r % 4:
// stored at row 16 b + r, a 16-lane group reads 16 consecutive rows, which with a row stride of
// 20 (mod 64) words or 36 words falls on 16 disjoint groups of four LDS banks.
__device__ __forceinline__ int perm_row(int x, int per) {
    return 16 * ((x % per) >> 2) + 4 * (x / per) + (x & 3);
}
// perm_row(col + j, per) for col a multiple of 8, j < 8 and per a multiple of 8: a per-lane base
// plus a compile-time offset for each j.
__device__ __forceinline__ int perm_base8(int col, int per) { return 4 * (col % per) + 4 * (col / per); }
__host__ __device__ constexpr int perm_off8(int j) { return 16 * (j >> 2) + (j & 3); }

// gfx950 LDS transpose read (ds_read_b64_tr_b16). Within each group of 16 lanes every lane points
// at 4 fp16 values (8 bytes, 8-byte aligned); lane i receives in slot j value i % 4 of the 8
// bytes that lane 4 j + i / 4 points at.
__device__ __forceinline__ half4 lds_read_tr16(const half_t* p) {
    typedef short short4v __attribute__((ext_vector_type(4)));
    typedef __attribute__((address_space(3))) short4v lds_short4;
    const short4v r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (lds_short4*)((__attribute__((address_space(3))) char*)p));
    return __builtin_bit_cast(half4, r);
}

// An MFMA operand whose 8 k-slots come from 8 rows of a row-major fp16 tile in LDS: lane i of
// 16-lane group g gets, for its row index x(i) = `cols` + (i / 4) * cstride + i % 4, the values
// tile[row(8 g + j)][x(i)] for j = 0..7, where the caller's `at(r)` gives the address of tile row
// r (after any row permutation). Two transpose reads, 4 rows each.
template <typename At>
__device__ __forceinline__ half8 lds_operand_tr(At at, int g, int lane16, int cols, int cstride) {
    const int j = lane16 >> 2, c = lane16 & 3;
    const half4 lo = lds_read_tr16(at(8 * g + j) + cols + c * cstride);
    const half4 hi = lds_read_tr16(at(8 * g + 4 + j) + cols + c * cstride);
    return half8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

// Pin v as an fp32 register value, so its later rounding to fp16 is a separate step that the
// compiler cannot fold into the multiply producing v (v_fma_mixlo_f16 rounds once). Every
// template variant of a kernel then rounds alike, as the reference rounds its fp32 dS.
__device__ __forceinline__ float pin_f32(float v) {
    asm volatile("" : "+v"(v));
    return v;
}

// sigmoid(g) = 1 / (1 + 2^(-g log2 e)), one v_exp_f32 and one v_rcp_f32
__device__ __forceinline__ float sigmoid_fast(float g) {
    return __builtin_amdgcn_rcpf(1.0f + exp2_fast(-kLog2e * g));
}

// Bias values of 16 consecutive keys (lo = keys 0..7, hi = 8..15) with key kk replaced by
// `masked` where its keep bit is clear but it lies inside Sk, and by `outside` past Sk. Works on
// the fp16 pairs: per pair a 32-bit select mask from the two keep bits (arithmetic shifts of
// the bit to all ones) and one bitfield insert, so a tile's masks are computed once for all its
// query blocks and a pair costs a few instructions instead of two compares and selects per key.
__device__ __forceinline__ uint32_t pair_mask(uint32_t bits, int p) {
    const uint32_t lo = (uint32_t)((int32_t)(bits << (31 - 2 * p)) >> 31);
    const uint32_t hi = (uint32_t)((int32_t)(bits << (30 - 2 * p)) >> 31);
    return (lo & 0xffffu) | (hi & 0xffff0000u);
}
__device__ __forceinline__ void fill_bias16(half8& lo, half8& hi, uint32_t keep, uint32_t inside,
                                            half_t masked, half_t outside) {
    typedef uint32_t u4 __attribute__((ext_vector_type(4)));
    u4 w[2] = {__builtin_bit_cast(u4, lo), __builtin_bit_cast(u4, hi)};
    const uint32_t mm = (uint32_t)__builtin_bit_cast(uint16_t, masked) * 0x10001u;
    const uint32_t oo = (uint32_t)__builtin_bit_cast(uint16_t, outside) * 0x10001u;
#pragma unroll
    for (int p = 0; p < 8; ++p) {
        const uint32_t im = pair_mask(inside, p), km = pair_mask(keep, p);
        const uint32_t f = (im & mm) | (~im & oo);
        w[p >> 2][p & 3] = (km & w[p >> 2][p & 3]) | (~km & f);
    }
    lo = __builtin_bit_cast(half8, w[0]);
    hi = __builtin_bit_cast(half8, w[1]);
}

__device__ __forceinline__ float wave_xor_sum4(float v) {
    // sum over the four lanes l, l^16, l^32, l^48 (one MFMA column's row groups)
    v += __shfl_xor(v, 16);
    v += __shfl_xor(v, 32);
    return v;
}

__device__ __forceinline__ float wave_xor_max4(float v) {
    v = fmaxf(v, __shfl_xor(v, 16));
    v = fmaxf(v, __shfl_xor(v, 32));
    return v;
}

// Work item of a 1-D launch, with consecutive items on the same XCD: the dispatcher deals
// workgroups round-robin over the 8 XCDs, so item i of XCD x is slot x's i-th workgroup.
// Neighbouring items share K/V (or weights) through that XCD's L2.
// Division of n < 2^31 by a runtime divisor 1 <= d < 2^31 as a multiply-high and a shift, so a
// work item's decomposition runs on the scalar unit instead of a VALU division sequence
// (Granlund and Montgomery's round-up method: mul = ceil(2^p / d), p = 31 + ceil(log2 d), exact
// for every n < 2^31; d = 1 has mul = 0).
struct FastDiv {
    uint32_t mul = 0, shift = 0, d = 1;
};
inline FastDiv fast_div(int64_t d) {
    FastDiv f;
    f.d = (uint32_t)(d < 1 ? 1 : d);
    if (f.d == 1) return f;
    uint32_t l = 0;
    while ((1ull << l) < f.d) ++l;
    f.mul = (uint32_t)(((1ull << (31 + l)) + f.d - 1) / f.d);
    f.shift = l - 1;
    return f;
}
__device__ __forceinline__ int fdiv(int n, FastDiv f) {
    return f.mul ? (int)(__umulhi((uint32_t)n, f.mul) >> f.shift) : n;
}

__device__ __forceinline__ int xcd_item(int linear, int count) {
    constexpr int kXcds = 8;
    const int x = linear % kXcds, s = linear / kXcds;
    const int per = count / kXcds, extra = count % kXcds;
    return x * per + (x < extra ? x : extra) + s;
}

// ---- host side ----------------------------------------------------------------------------

// Thread-local last error; every entry point returns through ok() or fail().
int fail(int code, const std::string& msg);
int ok();

inline int invalid(const std::string& msg) { return fail(CLK_INVALID_ARGUMENT, msg); }

int launch_status(const char* what);

// Records stage event i on stream s if a caller armed clk_set_stage_events with more than i.
void stage_mark(hipStream_t s, int i);

// Device LDS limit per workgroup, read once per device (a benign race, like the reference's
// per-device caches).
int shared_limit(int device);

inline int64_t elements(const clk_buffer* b) {
    int64_t n = 1;
    for (int i = 0; i < b->rank; ++i) n *= b->dims[i];
    return n;
}

inline bool is_rank(const clk_buffer* b, int r) { return b != nullptr && b->rank == r; }

inline bool same_shape(const clk_buffer* a, const clk_buffer* b) {
    if (a->rank != b->rank) return false;
    for (int i = 0; i < a->rank; ++i)
        if (a->dims[i] != b->dims[i]) return false;
    return true;
}

inline bool dims_are(const clk_buffer* b, int64_t d0, int64_t d1, int64_t d2) {
    return b->rank == 3 && b->dims[0] == d0 && b->dims[1] == d1 && b->dims[2] == d2;
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// The element-type check XLA's typed binding does before the handler runs.
int check_types(const char* what, const clk_buffer* const* bufs, const int* types, int n);

}  // namespace clk
