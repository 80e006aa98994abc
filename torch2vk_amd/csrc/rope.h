// Per-head RMSNorm + rotate-half RoPE for head_dim 128, one wave per head:
// lane l holds dims l and l + 64, which rotate together.  Shared by the decode
// attention prologue and the prefill chunk prologue so both produce the same
// q/k bits for a token at a given position.
//   inv_freq(l) = theta^(-2 l / 128)            (src/torch2vk/runtime/rope_table.py:109-119)
//   out[d] = n[d] cos - n[d + 64] sin, out[d + 64] = n[d + 64] cos + n[d] sin
//   (src/models/optimized_qwen3/shaders/rms_norm_rope_transpose_f16.py:97-143)
#pragma once

#include "common.h"

namespace t2h {

constexpr int ROPE_D = 128;

__device__ __forceinline__ void rope_cos_sin(int lane, int pos, float theta, float& cs, float& sn) {
    const float inv_freq = exp2f(-(2.0f * (float)lane / (float)ROPE_D) * log2f(theta));
    sincosf((float)pos * inv_freq, &sn, &cs);
}

__device__ __forceinline__ void norm_rope_pair(float x0, float x1, bool has_w, float w0, float w1, float eps,
                                               float cs, float sn, bool rope, float& r0, float& r1) {
    float n0 = x0, n1 = x1;
    if (has_w) {
        const float ss = wave_sum(x0 * x0 + x1 * x1);
        const float inv = 1.0f / sqrtf(ss / (float)ROPE_D + eps);
        n0 = x0 * inv * w0;
        n1 = x1 * inv * w1;
    }
    if (rope) {
        r0 = n0 * cs - n1 * sn;
        r1 = n1 * cs + n0 * sn;
    } else {
        r0 = n0;
        r1 = n1;
    }
}

}  // namespace t2h
