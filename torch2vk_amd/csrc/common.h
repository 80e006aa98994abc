// Device helpers shared by the gfx950 kernels of libt2h.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "t2h.h"

#define T2H_WAVE 64

namespace t2h {

// ---------------------------------------------------------------- numbers --

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t bits16) {
    return __uint_as_float(bits16 << 16);
}

typedef __bf16 t2h_bf16x2_t __attribute__((ext_vector_type(2)));
typedef float t2h_f32x2_t __attribute__((ext_vector_type(2)));

// fp32 -> bf16, round to nearest even, on the gfx950 converter
// (v_cvt_pk_bf16_f32: one instruction per two values, no branch; a NaN stays a NaN).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    const t2h_f32x2_t v = {lo, hi};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, t2h_bf16x2_t));
}

__device__ __forceinline__ uint32_t f32_to_bf16_bits(float v) {
    return (uint32_t)__builtin_bit_cast(unsigned short, (__bf16)v);
}

// IEEE binary16 -> fp32 (exact).
__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (unsigned short)(h & 0xffffu));
}

// fp32 -> binary16 bits, round to nearest even, subnormals kept.  Written out
// bit by bit so that it matches the CPU oracle exactly, independent of the
// hardware conversion's denormal mode.
__device__ __forceinline__ uint32_t f32_to_f16_bits_rne(float value) {
    uint32_t bits = __float_as_uint(value);
    const uint32_t sign = (bits >> 16) & 0x8000u;
    const uint32_t exp = (bits >> 23) & 0xffu;
    uint32_t mant = bits & 0x7fffffu;
    if (exp == 0xffu) return sign | 0x7c00u | (mant ? 0x200u : 0u);
    const int e = (int)exp - 127 + 15;
    if (e >= 31) return sign | 0x7c00u;
    if (e <= 0) {
        if (e < -10) return sign;
        mant |= 0x800000u;
        const uint32_t shift = (uint32_t)(14 - e);
        uint32_t half_mant = mant >> shift;
        const uint32_t rem = mant & ((1u << shift) - 1u);
        const uint32_t halfway = 1u << (shift - 1u);
        if (rem > halfway || (rem == halfway && (half_mant & 1u))) half_mant += 1u;
        return sign | half_mant;
    }
    uint32_t half = ((uint32_t)e << 10) | (mant >> 13);
    const uint32_t rem = mant & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (half & 1u))) half += 1u;
    return sign | half;
}

// Two-element dot products accumulated in fp32 (v_dot2_f32_bf16 / v_dot2_f32_f16):
// a and b each hold two 16-bit values, low half first.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a), __builtin_bit_cast(bf16x2_t, b), c,
                                           false);
}

__device__ __forceinline__ float dot2_f16(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, a), __builtin_bit_cast(f16x2_t, b), c, false);
}

// ------------------------------------------------------------- reductions --

// DPP move of a float within 16-lane rows (ctrl: quad_perm / row_mirror ...).
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, true));
}

// Exchange between lanes l and l ^ MASK (MASK 16 or 32) on v_permlane16_swap /
// v_permlane32_swap: VALU instructions, where __shfl_xor is an LDS-crossbar
// permute (ds_bpermute).  With operands (a, b), a lane with bit MASK clear gets
// (its a, the partner's a) and a lane with it set (the partner's b, its b).
template <int MASK>
__device__ __forceinline__ void lane_swap(float a, float b, float& r0, float& r1) {
    static_assert(MASK == 16 || MASK == 32, "swap across 16 or 32 lanes");
    const uint32_t ua = __float_as_uint(a), ub = __float_as_uint(b);
    if constexpr (MASK == 32) {
        const auto r = __builtin_amdgcn_permlane32_swap(ua, ub, false, false);
        r0 = __uint_as_float(r[0]);
        r1 = __uint_as_float(r[1]);
    } else {
        const auto r = __builtin_amdgcn_permlane16_swap(ua, ub, false, false);
        r0 = __uint_as_float(r[0]);
        r1 = __uint_as_float(r[1]);
    }
}

// x[l] + x[l ^ MASK] and max(x[l], x[l ^ MASK]) in every lane: the same values
// as x + __shfl_xor(x, MASK) (addition and max commute).
template <int MASK>
__device__ __forceinline__ float xor_sum(float x) {
    float r0, r1;
    lane_swap<MASK>(x, x, r0, r1);
    return r0 + r1;
}
template <int MASK>
__device__ __forceinline__ float xor_max(float x) {
    float r0, r1;
    lane_swap<MASK>(x, x, r0, r1);
    return fmaxf(r0, r1);
}

// Reduce-scatter of a pair across lanes l and l ^ MASK: the lane with bit MASK
// clear gets lo + the partner's lo, the other hi + the partner's hi.
template <int MASK>
__device__ __forceinline__ float xor_reduce_scatter(float lo, float hi) {
    float r0, r1;
    lane_swap<MASK>(lo, hi, r0, r1);
    return r0 + r1;
}

// ds_read_b64_tr_b16 (gfx950), 8 bytes per lane from LDS, transposed within each
// 16-lane group: with row(L) the four 16-bit elements at lane L's address, lane i
// receives element j of its result = row(4 j + i / 4)[i % 4], j = 0..3.
typedef short t2h_v4i16 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint2 lds_read_tr16_b64(const uint16_t* lds) {
    const t2h_v4i16 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (t2h_v4i16 __attribute__((address_space(3)))*)(lds));
    return __builtin_bit_cast(uint2, r);
}

// Sum over the 64 lanes of a wave; every lane gets the total.  Butterfly
// within each 16-lane row with DPP (xor 1, xor 2, half-row mirror, row
// mirror), then the four row totals are read out as scalars.
__device__ __forceinline__ float wave_sum(float v) {
    v += dpp_f32<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp_f32<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dpp_f32<0x141>(v);  // row_half_mirror
    v += dpp_f32<0x140>(v);  // row_mirror
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return (r0 + r1) + (r2 + r3);
}

// Max over the 64 lanes of a wave; every lane gets the result (same DPP
// pattern as wave_sum, no LDS round trips).
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_f32<0xB1>(v));   // quad_perm [1,0,3,2]
    v = fmaxf(v, dpp_f32<0x4E>(v));   // quad_perm [2,3,0,1]
    v = fmaxf(v, dpp_f32<0x141>(v));  // row_half_mirror
    v = fmaxf(v, dpp_f32<0x140>(v));  // row_mirror
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

// (score, token) argmax with the reference tie rule: higher score wins, equal
// scores go to the lower token id.
__device__ __forceinline__ bool better_pair(float ls, uint32_t lt, float rs, uint32_t rt) {
    return ls > rs || (ls == rs && lt < rt);
}

__device__ __forceinline__ void wave_argmax(float& score, uint32_t& token) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float os = __shfl_xor(score, off, T2H_WAVE);
        const uint32_t ot = (uint32_t)__shfl_xor((int)token, off, T2H_WAVE);
        if (better_pair(os, ot, score, token)) {
            score = os;
            token = ot;
        }
    }
}

// --------------------------------------------------------------- loads -----

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

// Streaming 16-byte load for weights that are read exactly once per pass.
__device__ __forceinline__ uint4 load_nt_u4(const void* p) {
    const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ float2 load_nt_f2(const float* p) {
    const f32x2_t v = __builtin_nontemporal_load(reinterpret_cast<const f32x2_t*>(p));
    return make_float2(v.x, v.y);
}

__device__ __forceinline__ uint4 load_u4(const void* p) { return *reinterpret_cast<const uint4*>(p); }

// Loads at 2-byte-aligned addresses (Q6_K blocks are 210 B and Q8_0 blocks
// 34 B, so their fields are only halfword aligned).  Under the HSA ABI the
// backend runs in unaligned-access mode and emits one global_load_dwordx4 /
// dwordx2 for these; the memory pipeline splits the access where it crosses
// a dword boundary.
__device__ __forceinline__ uint4 load_u4_ua(const uint8_t* p) {
    u32x4_t v;
    __builtin_memcpy(&v, p, 16);
    return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ uint2 load_u2_ua(const uint8_t* p) {
    uint2 v;
    __builtin_memcpy(&v, p, 8);
    return v;
}

__device__ __forceinline__ uint32_t load_u16(const uint8_t* p) {
    return *reinterpret_cast<const unsigned short*>(p);
}

// GELU(v) = v / 2 (1 + erf(v / sqrt 2)), erf by Abramowitz and Stegun 7.1.26 (|error| <= 1.5e-7), the
// approximation the reference's GELU shaders evaluate (src/models/quantized_qwen3_asr/shaders/gelu_f32.py:61-76):
// for z >= 0, erf(z) = 1 - q(t) e^(-z^2), t = 1 / (1 + p z), q a degree-5 polynomial in t without constant term.
// With z = |v| / sqrt 2, 1 + erf(v / sqrt 2) is 2 - q e^(-z^2) for v >= 0 and q e^(-z^2) for v < 0 (no
// cancellation for large negative v).  One reciprocal, one exp2 and 7 fused multiply-adds, against the ~30
// instructions of the library erff, which took a quarter of a bias + GELU GEMM of K 1024.
__device__ __forceinline__ float gelu_as(float v) {
    const float z = fabsf(v) * 0.70710678118654752f;
    const float t = __builtin_amdgcn_rcpf(fmaf(0.3275911f, z, 1.0f));
    const float q = t * fmaf(t, fmaf(t, fmaf(t, fmaf(t, 1.061405429f, -1.453152027f), 1.421413741f), -0.284496736f),
                             0.254829592f);
    const float qe = q * __builtin_amdgcn_exp2f(-1.4426950408889634f * z * z);
    return 0.5f * v * (v >= 0.0f ? 2.0f - qe : qe);
}

}  // namespace t2h

// Launch-result helper for the C-ABI layer.
#define T2H_LAUNCH_CHECK()                                     \
    do {                                                       \
        hipError_t _e = hipGetLastError();                     \
        if (_e != hipSuccess) return T2H_ERR_HIP_BASE + (int)_e; \
    } while (0)
