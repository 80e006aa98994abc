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
    const float* q;    // [n_seq * n, q_row]: head h at columns 128 h
    const float* k;    // [n_seq * n, k_row]
    const float* v;    // [n_seq * n, v_row]
    size_t q_row, k_row, v_row;
    const float* q_norm_w;
    const float* k_norm_w;
    float eps;
    float theta;       // <= 0: no RoPE
    int32_t start;     // position of each sequence's token 0
    uint32_t n, n_seq, nh, nk;
    uint16_t* q_out;   // [n_seq * n, nh, 128]
    uint16_t* k_cache; // [n_seq][s_cap, nk, 128]
    uint16_t* v_cache;
    size_t cache_seq;  // elements between two sequences' caches (s_cap * nk * 128)
};

constexpr int QK_HEADS_PER_WAVE = 8;

// A wave takes QK_HEADS_PER_WAVE of the q and k heads (q heads first) of one token: the RoPE factors of the
// token's position are computed once for all of them, and every head's loads are issued before any is used.
__global__ __launch_bounds__(256) void qk_norm_rope_cache_kernel(const QkRopeArgs a) {
    const uint32_t lane = threadIdx.x & 63;
    const uint64_t unit = (uint64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const uint32_t heads = a.nh + a.nk;
    const uint32_t groups = (heads + QK_HEADS_PER_WAVE - 1) / QK_HEADS_PER_WAVE;
    if (unit >= (uint64_t)a.n_seq * a.n * groups) return;
    const uint64_t row = unit / groups;  // the token's row of q|k|v and q_out
    const uint32_t h0 = (uint32_t)(unit - row * groups) * QK_HEADS_PER_WAVE;
    const uint32_t seq = (uint32_t)(row / a.n), tok = (uint32_t)(row - (uint64_t)seq * a.n);
    const int pos = a.start + (int)tok;
    const bool has_w = a.q_norm_w != nullptr;
    const float qw0 = has_w ? a.q_norm_w[lane] : 1.0f, qw1 = has_w ? a.q_norm_w[lane + 64] : 1.0f;
    const float kw0 = has_w ? a.k_norm_w[lane] : 1.0f, kw1 = has_w ? a.k_norm_w[lane + 64] : 1.0f;
    const bool rope = a.theta > 0.0f;
    float cs = 1.0f, sn = 0.0f;
    if (rope) rope_cos_sin((int)lane, pos, a.theta, cs, sn);
    float x0[QK_HEADS_PER_WAVE], x1[QK_HEADS_PER_WAVE];
    uint32_t vv[QK_HEADS_PER_WAVE];
#pragma unroll
    for (int j = 0; j < QK_HEADS_PER_WAVE; ++j) {
        const uint32_t hd = h0 + j < heads ? h0 + j : heads - 1;  // past the last head: re-read it, store nothing
        const bool is_q = hd < a.nh;
        const uint32_t h = is_q ? hd : hd - a.nh;
        const float* x = is_q ? a.q + row * a.q_row + (size_t)h * ROPE_D : a.k + row * a.k_row + (size_t)h * ROPE_D;
        x0[j] = x[lane];
        x1[j] = x[lane + 64];
        vv[j] = 0u;
        if (!is_q) {  // uniform across the wave
            const float* v = a.v + row * a.v_row + (size_t)h * ROPE_D;
            vv[j] = pack_bf16x2(v[2 * lane], v[2 * lane + 1]);
        }
    }
    uint16_t* kc = a.k_cache + (size_t)seq * a.cache_seq;
    uint16_t* vc = a.v_cache + (size_t)seq * a.cache_seq;
#pragma unroll
    for (int j = 0; j < QK_HEADS_PER_WAVE; ++j) {
        const uint32_t hd = h0 + j;
        if (hd >= heads) break;
        const bool is_q = hd < a.nh;
        const uint32_t h = is_q ? hd : hd - a.nh;
        float r0, r1;
        norm_rope_pair(x0[j], x1[j], has_w, is_q ? qw0 : kw0, is_q ? qw1 : kw1, a.eps, cs, sn, rope, r0, r1);
        if (is_q) {
            uint16_t* q = a.q_out + (row * a.nh + h) * ROPE_D;
            q[lane] = (uint16_t)f32_to_bf16_bits(r0);
            q[lane + 64] = (uint16_t)f32_to_bf16_bits(r1);
        } else {
            const size_t cache_row = ((size_t)pos * a.nk + h) * ROPE_D;
            kc[cache_row + lane] = (uint16_t)f32_to_bf16_bits(r0);
            kc[cache_row + lane + 64] = (uint16_t)f32_to_bf16_bits(r1);
            reinterpret_cast<uint32_t*>(vc + cache_row)[lane] = vv[j];
        }
    }
}

static int qk_norm_rope_launch(const float* q, uint64_t q_row, const float* k, uint64_t k_row, const float* v,
                               uint64_t v_row, const float* q_norm_w, const float* k_norm_w, float eps, float theta,
                               int32_t start, uint32_t n, uint32_t n_seq, uint32_t nh, uint32_t nk, uint32_t d,
                               void* q_out, void* k_cache, void* v_cache, uint32_t s_cap, void* stream) {
    if (!q || !k || !v || !q_out || !k_cache || !v_cache) return T2H_ERR_NULL;
    if ((q_norm_w == nullptr) != (k_norm_w == nullptr)) return T2H_ERR_NULL;
    if (d != ROPE_D) return T2H_ERR_UNSUPPORTED;
    if (nh == 0 || nk == 0 || n_seq == 0) return T2H_ERR_SHAPE;
    if (q_row < (uint64_t)nh * d || k_row < (uint64_t)nk * d || v_row < (uint64_t)nk * d) return T2H_ERR_SHAPE;
    if (start < 0 || (uint64_t)start + n > s_cap) return T2H_ERR_SHAPE;
    if (((reinterpret_cast<uintptr_t>(k_cache) | reinterpret_cast<uintptr_t>(v_cache)) & 3) != 0)
        return T2H_ERR_ALIGN;
    const uint64_t groups = (nh + nk + QK_HEADS_PER_WAVE - 1) / QK_HEADS_PER_WAVE;
    const uint64_t units = (uint64_t)n_seq * n * groups;
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
    a.n_seq = n_seq;
    a.nh = nh;
    a.nk = nk;
    a.q_out = reinterpret_cast<uint16_t*>(q_out);
    a.k_cache = reinterpret_cast<uint16_t*>(k_cache);
    a.v_cache = reinterpret_cast<uint16_t*>(v_cache);
    a.cache_seq = (size_t)s_cap * nk * d;
    hipLaunchKernelGGL(qk_norm_rope_cache_kernel, dim3((uint32_t)((units + 3) / 4)), dim3(256), 0,
                       reinterpret_cast<hipStream_t>(stream), a);
    T2H_LAUNCH_CHECK();
    return T2H_OK;
}

}  // namespace t2h

using namespace t2h;

extern "C" int t2h_qk_norm_rope_cache(const float* q, uint64_t q_row, const float* k, uint64_t k_row, const float* v,
                                      uint64_t v_row, const float* q_norm_w, const float* k_norm_w, float eps,
                                      float theta, int32_t start, uint32_t n, uint32_t nh, uint32_t nk, uint32_t d,
                                      void* q_out, void* k_cache, void* v_cache, uint32_t s_cap, void* stream) {
    return qk_norm_rope_launch(q, q_row, k, k_row, v, v_row, q_norm_w, k_norm_w, eps, theta, start, n, 1, nh, nk, d,
                               q_out, k_cache, v_cache, s_cap, stream);
}

extern "C" int t2h_qk_norm_rope_cache_seqs(const float* q, uint64_t q_row, const float* k, uint64_t k_row,
                                           const float* v, uint64_t v_row, const float* q_norm_w,
                                           const float* k_norm_w, float eps, float theta, int32_t start, uint32_t n,
                                           uint32_t n_seq, uint32_t nh, uint32_t nk, uint32_t d, void* q_out,
                                           void* k_cache, void* v_cache, uint32_t s_cap, void* stream) {
    return qk_norm_rope_launch(q, q_row, k, k_row, v, v_row, q_norm_w, k_norm_w, eps, theta, start, n, n_seq, nh, nk,
                               d, q_out, k_cache, v_cache, s_cap, stream);
}
