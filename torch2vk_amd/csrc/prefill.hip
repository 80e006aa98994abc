// Prefill chunk prologue of attention: for every token of a chunk, per-head
// RMSNorm + RoPE of q and k and the token-major KV cache write.
//
// Replaces, for a chunk of tokens at positions start .. start + n - 1:
//   RMS_NORM_ROPE_TOKEN_F32 / RMS_NORM_ROPE_TOKEN_F32_TO_F16
//       (src/models/optimized_qwen3/shaders/rms_norm_rope_token_f32.py:22-99)
//   TOKEN_MAJOR_KV_CACHE_WRITE_F16_PAIR / _TRIPLE and
//   TOKEN_MAJOR_VALUE_CACHE_WRITE_F32_TO_F16_PAIR / _TRIPLE
//       (src/models/optimized_qwen3/shaders/token_major_kv_cache_write_f16_pair.py:20-103)
// Input: the fp32 outputs of the chunk's q, k and v GEMMs, [n, *_row] each
// (column blocks of one buffer when the three weights share a GEMM).
// Output: q bf16 [n, nh, 128] for the flash-attention kernel, and k
// (normalised, rotated) and v as bf16 rows of the layer's cache
// [s_cap, nk, 128] at the tokens' positions.  One wave per (token, head); the
// math is the decode prologue's (rope.h), so a position's cached k is the same
// whether it was written by prefill or by a decode step.
#include "common.h"
#include "rope.h"

namespace t2h {

struct QkRopeArgs {
    const float* q;    // [n, q_row]: head h at columns 128 h
    const float* k;    // [n, k_row]
    const float* v;    // [n, v_row]
    size_t q_row, k_row, v_row;
    const float* q_norm_w;
    const float* k_norm_w;
    float eps;
    float theta;       // <= 0: no RoPE
    int32_t start;     // position of token 0
    uint32_t n, nh, nk;
    uint16_t* q_out;   // [n, nh, 128]
    uint16_t* k_cache; // [s_cap, nk, 128]
    uint16_t* v_cache;
};

__global__ __launch_bounds__(256) void qk_norm_rope_cache_kernel(const QkRopeArgs a) {
    const uint32_t lane = threadIdx.x & 63;
    const uint64_t unit = (uint64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const uint32_t heads = a.nh + a.nk;
    if (unit >= (uint64_t)a.n * heads) return;
    const uint32_t tok = (uint32_t)(unit / heads);
    const uint32_t hd = (uint32_t)(unit - (uint64_t)tok * heads);
    const int pos = a.start + (int)tok;
    const bool is_q = hd < a.nh;
    const uint32_t h = is_q ? hd : hd - a.nh;
    const float* x = is_q ? a.q + (size_t)tok * a.q_row + (size_t)h * ROPE_D
                          : a.k + (size_t)tok * a.k_row + (size_t)h * ROPE_D;
    const float x0 = x[lane], x1 = x[lane + 64];
    const float* nw = is_q ? a.q_norm_w : a.k_norm_w;
    const bool has_w = nw != nullptr;
    const float w0 = has_w ? nw[lane] : 1.0f, w1 = has_w ? nw[lane + 64] : 1.0f;
    const bool rope = a.theta > 0.0f;
    float cs = 1.0f, sn = 0.0f;
    if (rope) rope_cos_sin((int)lane, pos, a.theta, cs, sn);
    float r0, r1;
    norm_rope_pair(x0, x1, has_w, w0, w1, a.eps, cs, sn, rope, r0, r1);
    if (is_q) {
        uint16_t* q = a.q_out + ((size_t)tok * a.nh + h) * ROPE_D;
        q[lane] = (uint16_t)f32_to_bf16_bits(r0);
        q[lane + 64] = (uint16_t)f32_to_bf16_bits(r1);
        return;
    }
    const size_t cache_row = ((size_t)pos * a.nk + h) * ROPE_D;
    a.k_cache[cache_row + lane] = (uint16_t)f32_to_bf16_bits(r0);
    a.k_cache[cache_row + lane + 64] = (uint16_t)f32_to_bf16_bits(r1);
    const float* v = a.v + (size_t)tok * a.v_row + (size_t)h * ROPE_D;
    reinterpret_cast<uint32_t*>(a.v_cache + cache_row)[lane] = pack_bf16x2(v[2 * lane], v[2 * lane + 1]);
}

}  // namespace t2h

using namespace t2h;

extern "C" int t2h_qk_norm_rope_cache(const float* q, uint64_t q_row, const float* k, uint64_t k_row, const float* v,
                                      uint64_t v_row, const float* q_norm_w, const float* k_norm_w, float eps,
                                      float theta, int32_t start, uint32_t n, uint32_t nh, uint32_t nk, uint32_t d,
                                      void* q_out, void* k_cache, void* v_cache, uint32_t s_cap, void* stream) {
    if (!q || !k || !v || !q_out || !k_cache || !v_cache) return T2H_ERR_NULL;
    if ((q_norm_w == nullptr) != (k_norm_w == nullptr)) return T2H_ERR_NULL;
    if (d != ROPE_D) return T2H_ERR_UNSUPPORTED;
    if (nh == 0 || nk == 0) return T2H_ERR_SHAPE;
    if (q_row < (uint64_t)nh * d || k_row < (uint64_t)nk * d || v_row < (uint64_t)nk * d) return T2H_ERR_SHAPE;
    if (start < 0 || (uint64_t)start + n > s_cap) return T2H_ERR_SHAPE;
    if (((reinterpret_cast<uintptr_t>(k_cache) | reinterpret_cast<uintptr_t>(v_cache)) & 3) != 0)
        return T2H_ERR_ALIGN;
    const uint64_t units = (uint64_t)n * (nh + nk);
    if (units == 0) return T2H_OK;
    if ((units + 3) / 4 > 0x7fffffffu) return T2H_ERR_SHAPE;
    QkRopeArgs a;
    a.q = q;
    a.k = k;
    a.v = v;
    a.q_row = (size_t)q_row;
    a.k_row = (size_t)k_row;
    a.v_row = (size_t)v_row;
    a.q_norm_w = q_norm_w;
    a.k_norm_w = k_norm_w;
    a.eps = eps;
    a.theta = theta;
    a.start = start;
    a.n = n;
    a.nh = nh;
    a.nk = nk;
    a.q_out = reinterpret_cast<uint16_t*>(q_out);
    a.k_cache = reinterpret_cast<uint16_t*>(k_cache);
    a.v_cache = reinterpret_cast<uint16_t*>(v_cache);
    hipLaunchKernelGGL(qk_norm_rope_cache_kernel, dim3((uint32_t)((units + 3) / 4)), dim3(256), 0,
                       reinterpret_cast<hipStream_t>(stream), a);
    T2H_LAUNCH_CHECK();
    return T2H_OK;
}
