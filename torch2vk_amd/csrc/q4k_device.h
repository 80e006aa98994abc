// Q4_K decode building blocks shared by the GEMV kernels and the persistent
// decode-layers kernel: x staging in LDS as fp16 pair words, the per-lane
// header decode and the fp16 magic-number nibble dot product.
//
// Q4_K superblock (GGUF, 144 B per 256 values): fp16 d | fp16 dmin | 12 B of
// 6-bit scale/min codes | 128 B of nibbles; byte b of nibble group g holds
// value b of sub-block 2g (low nibble) and of sub-block 2g+1 (high nibble).
// Reference decoders: src/models/optimized_qwen3/shaders/linear_nobias_q4_k_matvec_f32.py:107-160,
// src/models/quantized_qwen3/shaders/embedding_q4_k_f32.py:79-110.
#pragma once

#include "common.h"

namespace t2h {

constexpr int cgcd(int a, int b) { return b == 0 ? a : cgcd(b, a % b); }

// ---------------------------------------------------------------- x in LDS --

__device__ __forceinline__ uint32_t f32_to_f16_bits(float v) {
    return (uint32_t)__builtin_bit_cast(unsigned short, (_Float16)v);
}

// A value known to be in a VGPR: VOP3 instructions (v_and_or_b32) take no
// literal operand on gfx9, so a mask held in a VGPR lets one v_and_or_b32 do
// the whole nibble expansion instead of an AND and an OR with literals.
__device__ __forceinline__ uint32_t in_vgpr(uint32_t v) {
    uint32_t r;
    asm("v_mov_b32 %0, %1" : "=v"(r) : "i"(v));
    return r;
}

// LDS layout of a staged x: fp16 pair words, 32 words (64 values) per group,
// each group followed by 4 pad words.  A lane's x slice is one whole group
// (superblock sb, nibble group g), and the pad puts the 8 lanes that share a
// 128-byte LDS cycle (4 groups of 2 superblocks) on distinct banks: without it
// every lane's slice starts on bank 0 and each 16-byte read is 8-way serialised.
__host__ __device__ constexpr int xp_words(int k) { return k / 2 + (k / 64) * 4; }
__device__ __forceinline__ int xp_word(int k) { return (k >> 1) + ((k >> 6) << 2); }

// Stage 4 consecutive x values (already bf16-exact) at element k: one fp16
// pair word (e0,e2) and one (e1,e3), and, through the 8 threads that hold one
// 32-value sub-block, that sub-block's sum (and, with xsum16, the sum of each
// 16 values, for Q6_K's scale groups).  All 8 threads of a sub-block call
// this together.
__device__ __forceinline__ void stage_x4(uint32_t* xp, float* xsum, int k, float v0, float v1, float v2, float v3,
                                         float* xsum16 = nullptr) {
    const uint32_t a = f32_to_f16_bits(v0) | (f32_to_f16_bits(v2) << 16);
    const uint32_t b = f32_to_f16_bits(v1) | (f32_to_f16_bits(v3) << 16);
    *reinterpret_cast<uint2*>(&xp[xp_word(k)]) = make_uint2(a, b);
    float s = (v0 + v1) + (v2 + v3);
    s += dpp_f32<0xB1>(s);  // quad_perm [1,0,3,2]: lane ^ 1
    s += dpp_f32<0x4E>(s);  // quad_perm [2,3,0,1]: lane ^ 2
    if (xsum16 != nullptr && ((k >> 2) & 3) == 0) xsum16[k >> 4] = s;  // the quad's 16 values
    s += dpp_f32<0x141>(s);  // row_half_mirror: a lane of the other quad of the 8, which holds that quad's sum
    if (((k >> 2) & 7) == 0) xsum[k >> 5] = s;
}

// One lane's x slice for one step: sub-blocks 2g and 2g+1 of superblock sb,
// as fp16 pair words, and 64 * each sub-block's sum.
struct XSlice16 {
    uint32_t lo[16];
    uint32_t hi[16];
    float sum_lo64;
    float sum_hi64;
};

__device__ __forceinline__ void load_xslice16(const uint32_t* xp, const float* xsum, int sb, int g, XSlice16& xs) {
    const uint32_t* p = xp + xp_word(sb * 256 + 64 * g);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint4 v = *reinterpret_cast<const uint4*>(p + 4 * i);
        xs.lo[4 * i] = v.x;
        xs.lo[4 * i + 1] = v.y;
        xs.lo[4 * i + 2] = v.z;
        xs.lo[4 * i + 3] = v.w;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint4 v = *reinterpret_cast<const uint4*>(p + 16 + 4 * i);
        xs.hi[4 * i] = v.x;
        xs.hi[4 * i + 1] = v.y;
        xs.hi[4 * i + 2] = v.z;
        xs.hi[4 * i + 3] = v.w;
    }
    xs.sum_lo64 = 64.0f * xsum[sb * 8 + 2 * g];
    xs.sum_hi64 = 64.0f * xsum[sb * 8 + 2 * g + 1];
}

// ------------------------------------------------------------ dot product --

// Per-lane constants of the header decode (nibble group g) and the masks.
struct Q4LaneConsts {
    uint32_t m_lo, m_hi;  // 0x000f000f / 0x00f000f0, in VGPRs
    int sh;               // 16 * (g & 1): byte pair of sub-blocks 2g, 2g+1 within a dword
    bool low;             // g < 2: 6-bit codes stored whole in bytes 4..11
    uint32_t mask_lo, hi_en;
    int sh_m;
};

__device__ __forceinline__ Q4LaneConsts q4k_lane_consts(int g) {
    Q4LaneConsts c;
    c.m_lo = in_vgpr(0x000f000fu);
    c.m_hi = in_vgpr(0x00f000f0u);
    c.sh = (g & 1) << 4;
    c.low = g < 2;
    c.mask_lo = c.low ? 0x3f3fu : 0x0f0fu;
    c.hi_en = c.low ? 0u : 0x3030u;
    c.sh_m = c.low ? c.sh : c.sh + 4;
    return c;
}

// Partial dot of one lane's 64 values of one superblock (nibble group g):
//   d*(sc_lo*sum(x q)_lo + sc_hi*sum(x q)_hi) - dmin*(m_lo*sum x_lo + m_hi*sum x_hi)
__device__ __forceinline__ float q4k_lane_dot(const uint4 hdr, const uint4 q0, const uint4 q1, const XSlice16& xs,
                                              const Q4LaneConsts& c) {
    constexpr uint32_t MAGIC = 0x54005400u;  // fp16 64.0 in both halves
    const float d = f16_bits_to_f32(hdr.x & 0xffffu);
    const float dmin = f16_bits_to_f32(hdr.x >> 16);
    // 6-bit scale/min codes of sub-blocks 2g and 2g+1 (get_scale_min_k4)
    const uint32_t src_s = c.low ? hdr.y : hdr.w;
    const uint32_t src_m = c.low ? hdr.z : hdr.w;
    const uint32_t S = ((src_s >> c.sh) & c.mask_lo) | ((hdr.y >> (c.sh + 2)) & c.hi_en);
    const uint32_t M = ((src_m >> c.sh_m) & c.mask_lo) | ((hdr.z >> (c.sh + 2)) & c.hi_en);
    const float sc_lo = (float)(S & 0xffu);
    const float sc_hi = (float)((S >> 8) & 0xffu);
    const float m_lo = (float)(M & 0xffu);
    const float m_hi = (float)((M >> 8) & 0xffu);

    float s_lo = 0.0f, s_hi = 0.0f;
    const uint32_t q[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
#pragma unroll
    for (int w = 0; w < 8; ++w) {
        const uint32_t b02 = q[w];       // bytes 0 and 2 of the word in the low bits of each half
        const uint32_t b13 = q[w] >> 8;  // bytes 1 and 3
        s_lo = dot2_f16((b02 & c.m_lo) | MAGIC, xs.lo[2 * w], s_lo);
        s_hi = dot2_f16((b02 & c.m_hi) | MAGIC, xs.hi[2 * w], s_hi);
        s_lo = dot2_f16((b13 & c.m_lo) | MAGIC, xs.lo[2 * w + 1], s_lo);
        s_hi = dot2_f16((b13 & c.m_hi) | MAGIC, xs.hi[2 * w + 1], s_hi);
    }
    const float xq_lo = 16.0f * (s_lo - xs.sum_lo64);
    const float xq_hi = s_hi - xs.sum_hi64;
    const float scaled = fmaf(sc_lo, xq_lo, sc_hi * xq_hi);
    const float mins = fmaf(m_lo, xs.sum_lo64, m_hi * xs.sum_hi64) * (1.0f / 64.0f);
    return fmaf(d, scaled, -dmin * mins);
}

__device__ __forceinline__ float silu(float g) { return g / (1.0f + expf(-g)); }

__device__ __forceinline__ float bf16_round(float v) { return bf16_bits_to_f32(f32_to_bf16_bits(v)); }

}  // namespace t2h
