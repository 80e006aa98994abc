// The reference's unfused operators, for callers that dispatch them by name.
//
// The decoder's own paths fuse these into their neighbours (RoPE and the q/k
// norms into attention or the chunk prologue, the residual adds into GEMM
// epilogues, the token select into one reduce).  A caller that runs the
// reference's per-op dispatch functions needs each of them on its own:
//   ROPE_TABLE_F32                       src/torch2vk/runtime/rope_table.py:32-122
//   RMS_NORM_ROPE_TRANSPOSE_F16          src/models/optimized_qwen3/shaders/rms_norm_rope_transpose_f16.py:22-145
//   RMS_NORM_ROPE_TOKEN_F32[_TO_F16]     src/models/optimized_qwen3/shaders/rms_norm_rope_token_f32.py:22-99
//   TOKEN_MAJOR_KV_CACHE_WRITE_F16_{PAIR,TRIPLE},
//   TOKEN_MAJOR_VALUE_CACHE_WRITE_F32_TO_F16_{PAIR,TRIPLE}
//                                        src/models/optimized_qwen3/shaders/token_major_kv_cache_write_f16_pair.py:20-103
//   QWEN3_TOKEN_SELECT_REDUCE_CHUNKS_F32 src/torch2vk/export/shaders/qwen3_token_select_reduce_f32.py:22-120
//   ADD_F32_PREFILL / ADD_F32_36         src/models/optimized_qwen3/shaders/add_f32_prefill.py:20-60
//   SLICE_LAST_TOKEN_F32_TO_F16          src/models/optimized_qwen3/shaders/slice_last_token_f32_to_f16.py:19-60
// The RoPE factors and the norm + rotation use the arithmetic of rope.h, the
// one the fused kernels use, so an fp32 table and these kernels give the
// fused path's q and k bits.
#include "common.h"
#include "rope.h"

namespace t2h {

// cos / sin [B, T, D] of positions start + t: inv_freq(d) = theta^(-2 (d mod D/2) / D).
__global__ __launch_bounds__(256) void rope_table_kernel(float* __restrict__ cos_out, float* __restrict__ sin_out,
                                                         uint32_t t_len, uint32_t d, uint64_t total,
                                                         uint32_t start, const int32_t* __restrict__ start_ptr,
                                                         float theta, float scaling) {
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= total) return;
    const uint32_t td = (uint32_t)(i % ((uint64_t)t_len * d));
    const uint32_t tok = td / d, dim = td - tok * d;
    const uint32_t l = dim % (d / 2);
    const int pos = (int)((start_ptr != nullptr ? (uint32_t)start_ptr[0] : start) + tok);
    float cs, sn;
    if (d == ROPE_D) {
        rope_cos_sin((int)l, pos, theta, cs, sn);
    } else {
        const float inv_freq = exp2f(-(2.0f * (float)l / (float)d) * log2f(theta));
        sincosf((float)pos * inv_freq, &sn, &cs);
    }
    cos_out[i] = cs * scaling;
    sin_out[i] = sn * scaling;
}

// Per-head RMSNorm over D = 128 then rotate-half RoPE from a table, one wave per (b, t, g) row: lane l holds
// dims l and l + 64.  x [B, T, G, D] (fp32 or bf16); out [B, T, G, D] or, transposed, [B, G, T, D].
struct NormRopeArgs {
    const void* x;
    const float* w;        // [D]
    const float* cos_t;    // [B, T, D]
    const float* sin_t;
    void* out;
    uint32_t b, t, g;
    float eps;
    int x_bf16, out_bf16, transpose;
};

__global__ __launch_bounds__(256) void rms_norm_rope_kernel(const NormRopeArgs a) {
    const uint32_t lane = threadIdx.x & 63;
    const uint64_t row = (uint64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const uint64_t rows = (uint64_t)a.b * a.t * a.g;
    if (row >= rows) return;
    const uint64_t bt = row / a.g;                 // (b, t)
    const uint32_t gi = (uint32_t)(row - bt * a.g);
    const uint64_t bi = bt / a.t;
    const uint32_t ti = (uint32_t)(bt - bi * a.t);
    const uint64_t xo = row * ROPE_D;
    float x0, x1;
    if (a.x_bf16) {
        const uint16_t* x = static_cast<const uint16_t*>(a.x) + xo;
        x0 = bf16_bits_to_f32(x[lane]);
        x1 = bf16_bits_to_f32(x[lane + 64]);
    } else {
        const float* x = static_cast<const float*>(a.x) + xo;
        x0 = x[lane];
        x1 = x[lane + 64];
    }
    const float* cs = a.cos_t + bt * ROPE_D;
    const float* sn = a.sin_t + bt * ROPE_D;
    const float c0 = cs[lane], s0 = sn[lane], c1 = cs[lane + 64], s1 = sn[lane + 64];
    const float ss = wave_sum(x0 * x0 + x1 * x1);
    const float inv = 1.0f / sqrtf(ss / (float)ROPE_D + a.eps);
    const float n0 = x0 * inv * a.w[lane];
    const float n1 = x1 * inv * a.w[lane + 64];
    const float r0 = n0 * c0 - n1 * s0;
    const float r1 = n1 * c1 + n0 * s1;
    const uint64_t oo = (a.transpose ? ((bi * a.g + gi) * a.t + ti) : row) * ROPE_D;
    if (a.out_bf16) {
        uint16_t* o = static_cast<uint16_t*>(a.out) + oo;
        o[lane] = (uint16_t)f32_to_bf16_bits(r0);
        o[lane + 64] = (uint16_t)f32_to_bf16_bits(r1);
    } else {
        float* o = static_cast<float*>(a.out) + oo;
        o[lane] = r0;
        o[lane + 64] = r1;
    }
}

// Token rows src [B, T, H, D] (fp32 or bf16) into up to 3 token-major bf16 caches [B, S_c, H, D] at positions
// pos[t]; a position outside a cache writes nothing there.  Two values per thread.
constexpr int KVW_MAX = 3;
struct KvWriteArgs {
    const void* src;
    const int64_t* pos;
    uint16_t* cache[KVW_MAX];
    uint32_t s_cap[KVW_MAX];
    uint32_t n_caches, b, t, hd;  // hd = H * D
    int src_bf16;
};

__global__ __launch_bounds__(256) void kv_cache_write_kernel(const KvWriteArgs a) {
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;  // pair index
    const uint64_t pairs = (uint64_t)a.b * a.t * a.hd / 2;
    if (i >= pairs) return;
    const uint64_t e = 2 * i;
    const uint64_t bt = e / a.hd;
    const uint32_t c = (uint32_t)(e - bt * a.hd);
    const uint64_t bi = bt / a.t;
    const uint32_t ti = (uint32_t)(bt - bi * a.t);
    uint32_t v;
    if (a.src_bf16) {
        v = reinterpret_cast<const uint32_t*>(a.src)[i];
    } else {
        const float2 f = reinterpret_cast<const float2*>(a.src)[i];
        v = pack_bf16x2(f.x, f.y);
    }
    const int64_t p = a.pos[ti];
    for (uint32_t k = 0; k < a.n_caches; ++k) {
        if (p < 0 || (uint64_t)p >= a.s_cap[k]) continue;
        uint16_t* row = a.cache[k] + ((bi * a.s_cap[k] + (uint64_t)p) * a.hd + c);
        *reinterpret_cast<uint32_t*>(row) = v;
    }
}

// Best (score, token) of each chunk of 1024 partials, ties to the lower token id.
__global__ __launch_bounds__(1024) void token_select_chunks_kernel(const float* __restrict__ scores,
                                                                   const uint32_t* __restrict__ tokens, uint32_t g,
                                                                   float* __restrict__ chunk_scores,
                                                                   uint32_t* __restrict__ chunk_tokens) {
    __shared__ float ss[16];
    __shared__ uint32_t st[16];
    const uint32_t i = blockIdx.x * 1024u + threadIdx.x;
    float bs = -3.4028234663852886e38f;
    uint32_t bt = 0xffffffffu;
    if (i < g) {
        bs = scores[i];
        bt = tokens[i];
    }
    wave_argmax(bs, bt);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) {
        ss[wave] = bs;
        st[wave] = bt;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float s = ss[0];
        uint32_t t = st[0];
        for (int w = 1; w < 16; ++w) {
            if (better_pair(ss[w], st[w], s, t)) {
                s = ss[w];
                t = st[w];
            }
        }
        chunk_scores[blockIdx.x] = s;
        chunk_tokens[blockIdx.x] = t;
    }
}

template <bool BF16>
__global__ __launch_bounds__(256) void add_kernel(const void* __restrict__ x, const void* __restrict__ y,
                                                  void* __restrict__ out, uint64_t n) {
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    if constexpr (BF16) {
        const float s = bf16_bits_to_f32(static_cast<const uint16_t*>(x)[i]) +
                        bf16_bits_to_f32(static_cast<const uint16_t*>(y)[i]);
        static_cast<uint16_t*>(out)[i] = (uint16_t)f32_to_bf16_bits(s);
    } else {
        static_cast<float*>(out)[i] = static_cast<const float*>(x)[i] + static_cast<const float*>(y)[i];
    }
}

// x fp32 [B, S, H] -> out [B, 1, H] (fp32 or bf16): row S - 1 of each batch.
__global__ __launch_bounds__(256) void slice_last_token_kernel(const float* __restrict__ x, void* __restrict__ out,
                                                               uint32_t s, uint32_t h, int out_bf16) {
    const uint32_t c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= h) return;
    const uint64_t bi = blockIdx.y;
    const float v = x[(bi * s + (s - 1)) * h + c];
    if (out_bf16)
        static_cast<uint16_t*>(out)[bi * h + c] = (uint16_t)f32_to_bf16_bits(v);
    else
        static_cast<float*>(out)[bi * h + c] = v;
}

static bool is_dtype(int d) { return d == T2H_DTYPE_F32 || d == T2H_DTYPE_BF16; }

}  // namespace t2h

using namespace t2h;

extern "C" int t2h_rope_table(float* cos_out, float* sin_out, uint32_t b, uint32_t t, uint32_t d, float theta,
                              uint32_t start_position, const int32_t* start_position_ptr, float attention_scaling,
                              void* stream) {
    if (!cos_out || !sin_out) return T2H_ERR_NULL;
    if (d == 0 || d % 2 || !(theta > 0.0f)) return T2H_ERR_SHAPE;
    const uint64_t total = (uint64_t)b * t * d;
    if (total == 0) return T2H_OK;
    if ((total + 255) / 256 > 0x7fffffffu) return T2H_ERR_SHAPE;
    hipLaunchKernelGGL(rope_table_kernel, dim3((uint32_t)((total + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                       cos_out, sin_out, t, d, total, start_position, start_position_ptr, theta, attention_scaling);
    T2H_LAUNCH_CHECK();
    return T2H_OK;
}

extern "C" int t2h_rms_norm_rope(const void* x, int x_dtype, const float* weight, const float* cos_table,
                                 const float* sin_table, void* out, int out_dtype, uint32_t b, uint32_t t, uint32_t g,
                                 uint32_t d, int transpose_out, float eps, void* stream) {
    if (!x || !weight || !cos_table || !sin_table || !out) return T2H_ERR_NULL;
    if (!is_dtype(x_dtype) || !is_dtype(out_dtype)) return T2H_ERR_DTYPE;
    if (d != ROPE_D) return T2H_ERR_UNSUPPORTED;
    const uint64_t rows = (uint64_t)b * t * g;
    if (rows == 0) return T2H_OK;
    if ((rows + 3) / 4 > 0x7fffffffu) return T2H_ERR_SHAPE;
    NormRopeArgs a;
    a.x = x;
    a.w = weight;
    a.cos_t = cos_table;
    a.sin_t = sin_table;
    a.out = out;
    a.b = b;
    a.t = t;
    a.g = g;
    a.eps = eps;
    a.x_bf16 = x_dtype == T2H_DTYPE_BF16;
    a.out_bf16 = out_dtype == T2H_DTYPE_BF16;
    a.transpose = transpose_out != 0;
    hipLaunchKernelGGL(rms_norm_rope_kernel, dim3((uint32_t)((rows + 3) / 4)), dim3(256), 0, (hipStream_t)stream, a);
    T2H_LAUNCH_CHECK();
    return T2H_OK;
}

extern "C" int t2h_kv_cache_write(const void* src, int src_dtype, const int64_t* positions, uint32_t n_caches,
                                  void* const* caches, const uint32_t* s_caps, uint32_t b, uint32_t t, uint32_t h,
                                  uint32_t d, void* stream) {
    if (!src || !positions || !caches || !s_caps) return T2H_ERR_NULL;
    if (!is_dtype(src_dtype)) return T2H_ERR_DTYPE;
    if (n_caches == 0 || n_caches > (uint32_t)KVW_MAX) return T2H_ERR_ARG;
    if (d == 0 || ((uint64_t)h * d) % 2) return T2H_ERR_SHAPE;
    if (reinterpret_cast<uintptr_t>(src) % (src_dtype == T2H_DTYPE_BF16 ? 4 : 8)) return T2H_ERR_ALIGN;
    KvWriteArgs a = {};
    for (uint32_t k = 0; k < n_caches; ++k) {
        if (!caches[k]) return T2H_ERR_NULL;
        if (reinterpret_cast<uintptr_t>(caches[k]) % 4) return T2H_ERR_ALIGN;
        a.cache[k] = static_cast<uint16_t*>(caches[k]);
        a.s_cap[k] = s_caps[k];
    }
    a.src = src;
    a.pos = positions;
    a.n_caches = n_caches;
    a.b = b;
    a.t = t;
    a.hd = h * d;
    a.src_bf16 = src_dtype == T2H_DTYPE_BF16;
    const uint64_t pairs = (uint64_t)b * t * h * d / 2;
    if (pairs == 0) return T2H_OK;
    if ((pairs + 255) / 256 > 0x7fffffffu) return T2H_ERR_SHAPE;
    hipLaunchKernelGGL(kv_cache_write_kernel, dim3((uint32_t)((pairs + 255) / 256)), dim3(256), 0,
                       (hipStream_t)stream, a);
    T2H_LAUNCH_CHECK();
    return T2H_OK;
}

extern "C" int t2h_token_select_chunks(const float* scores, const uint32_t* tokens, uint32_t g, float* chunk_scores,
                                       uint32_t* chunk_tokens, void* stream) {
    if (!scores || !tokens || !chunk_scores || !chunk_tokens) return T2H_ERR_NULL;
    if (g == 0) return T2H_ERR_SHAPE;
    hipLaunchKernelGGL(token_select_chunks_kernel, dim3((g + 1023) / 1024), dim3(1024), 0, (hipStream_t)stream, scores,
                       tokens, g, chunk_scores, chunk_tokens);
    T2H_LAUNCH_CHECK();
    return T2H_OK;
}

extern "C" int t2h_add(const void* x, const void* y, void* out, int dtype, uint64_t n, void* stream) {
    if (!x || !y || !out) return T2H_ERR_NULL;
    if (!is_dtype(dtype)) return T2H_ERR_DTYPE;
    if (n == 0) return T2H_OK;
    if ((n + 255) / 256 > 0x7fffffffu) return T2H_ERR_SHAPE;
    const dim3 grid((uint32_t)((n + 255) / 256));
    if (dtype == T2H_DTYPE_BF16)
        hipLaunchKernelGGL(add_kernel<true>, grid, dim3(256), 0, (hipStream_t)stream, x, y, out, n);
    else
        hipLaunchKernelGGL(add_kernel<false>, grid, dim3(256), 0, (hipStream_t)stream, x, y, out, n);
    T2H_LAUNCH_CHECK();
    return T2H_OK;
}

extern "C" int t2h_slice_last_token(const float* x, void* out, int out_dtype, uint32_t b, uint32_t s, uint32_t h,
                                    void* stream) {
    if (!x || !out) return T2H_ERR_NULL;
    if (!is_dtype(out_dtype)) return T2H_ERR_DTYPE;
    if (s == 0 || b > 65535) return T2H_ERR_SHAPE;
    if (b == 0 || h == 0) return T2H_OK;
    hipLaunchKernelGGL(slice_last_token_kernel, dim3((h + 255) / 256, b), dim3(256), 0, (hipStream_t)stream, x, out, s,
                       h, out_dtype == T2H_DTYPE_BF16 ? 1 : 0);
    T2H_LAUNCH_CHECK();
    return T2H_OK;
}
