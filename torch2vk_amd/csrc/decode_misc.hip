// Small decode-step kernels: embedding gather, greedy token select, token
// store, standalone RMSNorm and SwiGLU.
//
//   EMBEDDING_Q4_K_F32                   src/models/quantized_qwen3/shaders/embedding_q4_k_f32.py:62-121
//   QWEN3_TOKEN_SELECT_REDUCE_{CHUNKS_,}F32  src/torch2vk/export/shaders/qwen3_token_select_reduce_f32.py:22-241
//   QWEN3_TOKEN_STORE_EOS_F32            src/models/optimized_qwen3/shaders/qwen3_token_store_eos_f32.py:21-140
//   RMS_NORM_MUL_F16_F32                 src/models/optimized_qwen3/shaders/rms_norm_mul_f16_f32.py:22-115
//   SWIGLU_F16                           src/models/optimized_qwen3/shaders/swiglu_f16.py:20-81
#include <type_traits>

#include "common.h"

namespace t2h {

// One block per token: dequantise the token's Q4_K embedding row into fp32.
// Thread t handles nibble group (t & 3) of superblock (t >> 2): one 16-B
// header and 32 B of nibbles -> 64 values, written as 16 float4 stores.
__device__ __forceinline__ void embed_q4_k_row(const uint8_t* __restrict__ w, int64_t id, uint32_t dim, uint64_t vocab,
                                               float* __restrict__ out_row) {
    if (id < 0 || (uint64_t)id >= vocab) id = 0;  // the host validates host-side ids; device ids are clamped
    const uint32_t nsb = dim / 256;
    const uint8_t* row = w + (uint64_t)id * nsb * 144;
    for (uint32_t item = threadIdx.x; item < nsb * 4; item += blockDim.x) {
        const uint32_t sb = item >> 2;
        const int g = item & 3;
        const uint8_t* blk = row + (size_t)sb * 144;
        const uint4 hdr = *reinterpret_cast<const uint4*>(blk);
        const uint4 q0 = *reinterpret_cast<const uint4*>(blk + 16 + 32 * g);
        const uint4 q1 = *reinterpret_cast<const uint4*>(blk + 32 + 32 * g);
        const float d = f16_bits_to_f32(hdr.x & 0xffffu);
        const float dmin = f16_bits_to_f32(hdr.x >> 16);
        const uint8_t* sc8 = blk + 4;
        uint32_t sc[2], m[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int j = 2 * g + h;
            if (j < 4) {
                sc[h] = sc8[j] & 63u;
                m[h] = sc8[4 + j] & 63u;
            } else {
                sc[h] = (sc8[8 + j - 4] & 15u) | ((uint32_t)(sc8[j - 4] >> 6) << 4);
                m[h] = ((uint32_t)sc8[8 + j - 4] >> 4) | ((uint32_t)(sc8[4 + j - 4] >> 6) << 4);
            }
        }
        const uint32_t q[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
        float* o = out_row + sb * 256 + 64 * g;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const float a = d * (float)sc[h];
            const float b = dmin * (float)m[h];
#pragma unroll
            for (int c = 0; c < 8; ++c) {
                // (d*sc)*q - dmin*m with no contraction: the decoders' exact fp32 order
                const uint32_t wq = h ? (q[c] >> 4) : q[c];
                float4 v;
                v.x = __fsub_rn(__fmul_rn(a, (float)(wq & 15u)), b);
                v.y = __fsub_rn(__fmul_rn(a, (float)((wq >> 8) & 15u)), b);
                v.z = __fsub_rn(__fmul_rn(a, (float)((wq >> 16) & 15u)), b);
                v.w = __fsub_rn(__fmul_rn(a, (float)((wq >> 24) & 15u)), b);
                *reinterpret_cast<float4*>(o + 32 * h + 4 * c) = v;
            }
        }
    }
}

__global__ __launch_bounds__(256) void embedding_q4_k_kernel(const uint8_t* __restrict__ w,
                                                             const int64_t* __restrict__ ids, uint32_t dim,
                                                             uint64_t vocab, float* __restrict__ out) {
    embed_q4_k_row(w, ids[blockIdx.x], dim, vocab, out + (uint64_t)blockIdx.x * dim);
}

// One decode step's embedding for several sequences (a decoder group): block b embeds sequence b's next
// token into its own hidden row.
constexpr int SEQS_MAX = 4;
struct EmbedSeqsArgs {
    const int64_t* ids[SEQS_MAX];
    float* out[SEQS_MAX];
};

__global__ __launch_bounds__(256) void embedding_q4_k_seqs_kernel(const uint8_t* __restrict__ w, uint32_t dim,
                                                                  uint64_t vocab, const EmbedSeqsArgs a) {
    embed_q4_k_row(w, a.ids[blockIdx.x][0], dim, vocab, a.out[blockIdx.x]);
}

// Reduce G (score, token) partials to one greedy token; flag EOS.
__global__ __launch_bounds__(1024) void token_select_kernel(const float* __restrict__ scores,
                                                            const uint32_t* __restrict__ tokens, uint32_t g,
                                                            const int64_t* __restrict__ eos, uint32_t n_eos,
                                                            int64_t* __restrict__ next_token,
                                                            uint32_t* __restrict__ done) {
    __shared__ float ss[16];
    __shared__ uint32_t st[16];
    float bs = -3.4028234663852886e38f;
    uint32_t bt = 0xffffffffu;
    for (uint32_t i = threadIdx.x; i < g; i += blockDim.x) {
        if (better_pair(scores[i], tokens[i], bs, bt)) {
            bs = scores[i];
            bt = tokens[i];
        }
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
        for (int i = 1; i < (int)(blockDim.x >> 6); ++i) {
            if (better_pair(ss[i], st[i], s, t)) {
                s = ss[i];
                t = st[i];
            }
        }
        next_token[0] = (int64_t)t;
        uint32_t is_done = 0;
        for (uint32_t i = 0; i < n_eos; ++i) is_done |= ((int64_t)t == eos[i]) ? 1u : 0u;
        if (done) done[0] = is_done;
    }
}

// generated_tokens[index] = next_token; length = index + 1; stop on EOS.
// index comes from token_index_ptr (device) when given, else token_index.
// advance (optional, device) is incremented after a store: the caller's
// cache-position counter for graph-replayed decode loops.
__global__ void token_store_kernel(const int64_t* __restrict__ next_token, const uint32_t* __restrict__ done,
                                   int64_t* __restrict__ generated, uint32_t g, uint32_t* __restrict__ length,
                                   uint32_t* __restrict__ stopped, uint32_t stop_on_eos,
                                   const uint32_t* __restrict__ token_index_ptr, uint32_t token_index,
                                   int32_t* __restrict__ advance) {
    const uint32_t index = token_index_ptr ? *token_index_ptr : token_index;
    if (advance) advance[0] += 1;
    if (index >= g) return;
    if (stop_on_eos && stopped[0] != 0u) return;
    generated[index] = next_token[0];
    length[0] = index + 1u;
    if (stop_on_eos && done && done[0] != 0u) stopped[0] = 1u;
}

// Greedy select fused with the token store: one launch per decode step for
// both QWEN3_TOKEN_SELECT_REDUCE_F32 and QWEN3_TOKEN_STORE_EOS_F32.
__device__ __forceinline__ void token_select_store_block(
    const float* __restrict__ scores, const uint32_t* __restrict__ tokens, uint32_t g,
    const int64_t* __restrict__ eos, uint32_t n_eos, int64_t* __restrict__ next_token, uint32_t* __restrict__ done,
    int64_t* __restrict__ generated, uint32_t gen_cap, uint32_t* __restrict__ length, uint32_t* __restrict__ stopped,
    uint32_t stop_on_eos, int32_t* __restrict__ advance) {
    __shared__ float ss[16];
    __shared__ uint32_t st[16];
    float bs = -3.4028234663852886e38f;
    uint32_t bt = 0xffffffffu;
    for (uint32_t i = threadIdx.x; i < g; i += blockDim.x) {
        if (better_pair(scores[i], tokens[i], bs, bt)) {
            bs = scores[i];
            bt = tokens[i];
        }
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
        for (int i = 1; i < (int)(blockDim.x >> 6); ++i) {
            if (better_pair(ss[i], st[i], s, t)) {
                s = ss[i];
                t = st[i];
            }
        }
        next_token[0] = (int64_t)t;
        uint32_t is_done = 0;
        for (uint32_t i = 0; i < n_eos; ++i) is_done |= ((int64_t)t == eos[i]) ? 1u : 0u;
        if (done) done[0] = is_done;
        if (advance) advance[0] += 1;
        const uint32_t index = length[0];
        if (index < gen_cap && !(stop_on_eos && stopped[0] != 0u)) {
            generated[index] = (int64_t)t;
            length[0] = index + 1u;
            if (stop_on_eos && is_done) stopped[0] = 1u;
        }
    }
}

__global__ __launch_bounds__(1024) void token_select_store_kernel(
    const float* __restrict__ scores, const uint32_t* __restrict__ tokens, uint32_t g,
    const int64_t* __restrict__ eos, uint32_t n_eos, int64_t* __restrict__ next_token, uint32_t* __restrict__ done,
    int64_t* __restrict__ generated, uint32_t gen_cap, uint32_t* __restrict__ length, uint32_t* __restrict__ stopped,
    uint32_t stop_on_eos, int32_t* __restrict__ advance) {
    token_select_store_block(scores, tokens, g, eos, n_eos, next_token, done, generated, gen_cap, length, stopped,
                             stop_on_eos, advance);
}

// The select + store of several sequences (a decoder group's step): block b runs sequence b's, exactly as
// its own token_select_store_kernel launch would.
struct SelectStoreSeqsArgs {
    const float* scores[SEQS_MAX];
    const uint32_t* tokens[SEQS_MAX];
    int64_t* next_token[SEQS_MAX];
    uint32_t* done[SEQS_MAX];
    int64_t* generated[SEQS_MAX];
    uint32_t* length[SEQS_MAX];
    uint32_t* stopped[SEQS_MAX];
    int32_t* advance[SEQS_MAX];
};

__global__ __launch_bounds__(1024) void token_select_store_seqs_kernel(uint32_t g, const int64_t* __restrict__ eos,
                                                                       uint32_t n_eos, uint32_t gen_cap,
                                                                       uint32_t stop_on_eos,
                                                                       const SelectStoreSeqsArgs a) {
    const uint32_t b = blockIdx.x;
    token_select_store_block(a.scores[b], a.tokens[b], g, eos, n_eos, a.next_token[b], a.done[b], a.generated[b],
                             gen_cap, a.length[b], a.stopped[b], stop_on_eos, a.advance[b]);
}

// rows x H RMSNorm; x and out are fp32 or bf16, weight fp32.
template <bool XBF16, bool OBF16>
__global__ __launch_bounds__(256) void rms_norm_kernel(const void* __restrict__ xv, const float* __restrict__ w,
                                                       void* __restrict__ outv, uint32_t h, float eps) {
    __shared__ float red[4];
    const uint64_t base = (uint64_t)blockIdx.x * h;
    auto ld = [&](uint32_t i) -> float {
        if constexpr (XBF16) return bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(xv)[base + i]);
        else return reinterpret_cast<const float*>(xv)[base + i];
    };
    float ss = 0.0f;
    for (uint32_t i = threadIdx.x; i < h; i += 256) {
        const float v = ld(i);
        ss = fmaf(v, v, ss);
    }
    ss = wave_sum(ss);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    const float total = red[0] + red[1] + red[2] + red[3];
    const float inv = 1.0f / sqrtf(total / (float)h + eps);
    for (uint32_t i = threadIdx.x; i < h; i += 256) {
        const float v = ld(i) * inv * w[i];
        if constexpr (OBF16) reinterpret_cast<uint16_t*>(outv)[base + i] = (uint16_t)f32_to_bf16_bits(v);
        else reinterpret_cast<float*>(outv)[base + i] = v;
    }
}

// RMSNorm of fp32 rows of NCH * 1024 values: each thread keeps its NCH float4 of the row in registers, so the
// row is read from memory once, with 16-byte loads, and written with 8- (bf16) or 16-byte (fp32) stores.
template <int NCH, bool OBF16>
__global__ __launch_bounds__(256) void rms_norm_rows_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                            void* __restrict__ outv, uint32_t h, float eps) {
    __shared__ float red[4];
    const uint64_t base = (uint64_t)blockIdx.x * h;
    const float4* xr = reinterpret_cast<const float4*>(x + base);
    float4 v[NCH];
    float ss = 0.0f;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        v[c] = xr[c * 256 + threadIdx.x];
        ss = fmaf(v[c].x, v[c].x, ss);
        ss = fmaf(v[c].y, v[c].y, ss);
        ss = fmaf(v[c].z, v[c].z, ss);
        ss = fmaf(v[c].w, v[c].w, ss);
    }
    ss = wave_sum(ss);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    const float total = red[0] + red[1] + red[2] + red[3];
    const float inv = 1.0f / sqrtf(total / (float)h + eps);
    const float4* wr = reinterpret_cast<const float4*>(w);
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        const uint32_t i4 = c * 256 + threadIdx.x;
        const float4 wv = wr[i4];
        const float4 y = make_float4(v[c].x * inv * wv.x, v[c].y * inv * wv.y, v[c].z * inv * wv.z,
                                     v[c].w * inv * wv.w);
        if constexpr (OBF16)
            reinterpret_cast<uint2*>(outv)[base / 4 + i4] = make_uint2(pack_bf16x2(y.x, y.y), pack_bf16x2(y.z, y.w));
        else
            reinterpret_cast<float4*>(outv)[base / 4 + i4] = y;
    }
}

template <bool GBF16>
__global__ void swiglu_kernel(const void* __restrict__ gate, const void* __restrict__ up,
                              uint16_t* __restrict__ out, uint64_t n) {
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    float g, u;
    if constexpr (GBF16) {
        g = bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(gate)[i]);
        u = bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(up)[i]);
    } else {
        g = reinterpret_cast<const float*>(gate)[i];
        u = reinterpret_cast<const float*>(up)[i];
    }
    out[i] = (uint16_t)f32_to_bf16_bits(g / (1.0f + expf(-g)) * u);
}

}  // namespace t2h

using namespace t2h;

extern "C" int t2h_embedding_q4_k(const void* w, uint64_t vocab, const int64_t* ids, uint32_t n_ids, uint32_t dim,
                                  float* out, void* stream) {
    if (!w || !ids || !out) return T2H_ERR_NULL;
    if (dim == 0 || dim % 256 != 0 || vocab == 0) return T2H_ERR_SHAPE;
    // 16-B superblock loads and float4 stores
    if (reinterpret_cast<uintptr_t>(w) % 16 || reinterpret_cast<uintptr_t>(out) % 16) return T2H_ERR_ALIGN;
    if (n_ids == 0) return T2H_OK;
    hipLaunchKernelGGL(embedding_q4_k_kernel, dim3(n_ids), dim3(256), 0, (hipStream_t)stream,
                       (const uint8_t*)w, ids, dim, vocab, out);
    T2H_LAUNCH_CHECK();
    return T2H_OK;
}

extern "C" int t2h_token_select(const float* scores, const uint32_t* tokens, uint32_t g, const int64_t* eos,
                                uint32_t n_eos, int64_t* next_token, uint32_t* done, void* stream) {
    if (!scores || !tokens || !next_token) return T2H_ERR_NULL;
    if (n_eos && !eos) return T2H_ERR_NULL;
    if (g == 0) return T2H_ERR_SHAPE;
    hipLaunchKernelGGL(token_select_kernel, dim3(1), dim3(1024), 0, (hipStream_t)stream, scores, tokens, g, eos,
                       n_eos, next_token, done);
    T2H_LAUNCH_CHECK();
    return T2H_OK;
}

extern "C" int t2h_token_select_store(const float* scores, const uint32_t* tokens, uint32_t g,
                                      const int64_t* eos, uint32_t n_eos, int64_t* next_token, uint32_t* done,
                                      int64_t* generated, uint32_t gen_cap, uint32_t* length, uint32_t* stopped,
                                      uint32_t stop_on_eos, int32_t* advance, void* stream) {
    if (!scores || !tokens || !next_token || !generated || !length || !stopped) return T2H_ERR_NULL;
    if (n_eos && !eos) return T2H_ERR_NULL;
    if (g == 0) return T2H_ERR_SHAPE;
    hipLaunchKernelGGL(token_select_store_kernel, dim3(1), dim3(1024), 0, (hipStream_t)stream, scores, tokens, g, eos,
                       n_eos, next_token, done, generated, gen_cap, length, stopped, stop_on_eos, advance);
    T2H_LAUNCH_CHECK();
    return T2H_OK;
}

extern "C" int t2h_embedding_q4_k_seqs(uint32_t n_seq, const void* w, uint64_t vocab, const int64_t* const* ids,
                                       uint32_t dim, float* const* out, void* stream) {
    if (!w || !ids || !out) return T2H_ERR_NULL;
    if (n_seq == 0 || n_seq > (uint32_t)SEQS_MAX) return T2H_ERR_ARG;
    if (dim == 0 || dim % 256 != 0 || vocab == 0) return T2H_ERR_SHAPE;
    if (reinterpret_cast<uintptr_t>(w) % 16) return T2H_ERR_ALIGN;  // 16-B superblock loads
    EmbedSeqsArgs a = {};
    for (uint32_t i = 0; i < n_seq; ++i) {
        if (!ids[i] || !out[i]) return T2H_ERR_NULL;
        if (reinterpret_cast<uintptr_t>(out[i]) % 16) return T2H_ERR_ALIGN;  // float4 stores
        a.ids[i] = ids[i];
        a.out[i] = out[i];
    }
    hipLaunchKernelGGL(embedding_q4_k_seqs_kernel, dim3(n_seq), dim3(256), 0, (hipStream_t)stream,
                       (const uint8_t*)w, dim, vocab, a);
    T2H_LAUNCH_CHECK();
    return T2H_OK;
}

extern "C" int t2h_token_select_store_seqs(uint32_t n_seq, const float* const* scores, const uint32_t* const* tokens,
                                           uint32_t g, const int64_t* eos, uint32_t n_eos, int64_t* const* next_token,
                                           uint32_t* const* done, int64_t* const* generated, uint32_t gen_cap,
                                           uint32_t* const* length, uint32_t* const* stopped, uint32_t stop_on_eos,
                                           int32_t* const* advance, void* stream) {
    if (!scores || !tokens || !next_token || !done || !generated || !length || !stopped || !advance)
        return T2H_ERR_NULL;
    if (n_seq == 0 || n_seq > (uint32_t)SEQS_MAX) return T2H_ERR_ARG;
    if (n_eos && !eos) return T2H_ERR_NULL;
    if (g == 0) return T2H_ERR_SHAPE;
    SelectStoreSeqsArgs a = {};
    for (uint32_t i = 0; i < n_seq; ++i) {
        if (!scores[i] || !tokens[i] || !next_token[i] || !generated[i] || !length[i] || !stopped[i])
            return T2H_ERR_NULL;
        a.scores[i] = scores[i];
        a.tokens[i] = tokens[i];
        a.next_token[i] = next_token[i];
        a.done[i] = done[i];          // may be null, as in t2h_token_select_store
        a.generated[i] = generated[i];
        a.length[i] = length[i];
        a.stopped[i] = stopped[i];
        a.advance[i] = advance[i];    // may be null
    }
    hipLaunchKernelGGL(token_select_store_seqs_kernel, dim3(n_seq), dim3(1024), 0, (hipStream_t)stream, g, eos, n_eos,
                       gen_cap, stop_on_eos, a);
    T2H_LAUNCH_CHECK();
    return T2H_OK;
}

extern "C" int t2h_token_store(const int64_t* next_token, const uint32_t* done, int64_t* generated, uint32_t g,
                               uint32_t* length, uint32_t* stopped, uint32_t stop_on_eos,
                               const uint32_t* token_index_ptr, uint32_t token_index, int32_t* advance,
                               void* stream) {
    if (!next_token || !generated || !length || !stopped) return T2H_ERR_NULL;
    hipLaunchKernelGGL(token_store_kernel, dim3(1), dim3(1), 0, (hipStream_t)stream, next_token, done, generated, g,
                       length, stopped, stop_on_eos, token_index_ptr, token_index, advance);
    T2H_LAUNCH_CHECK();
    return T2H_OK;
}

extern "C" int t2h_rms_norm(const void* x, int x_dtype, const float* w, void* out, int out_dtype, uint32_t rows,
                            uint32_t h, float eps, void* stream) {
    if (!x || !w || !out) return T2H_ERR_NULL;
    if (h == 0) return T2H_ERR_SHAPE;
    if (rows == 0) return T2H_OK;
    hipStream_t s = (hipStream_t)stream;
    const bool xb = x_dtype == T2H_DTYPE_BF16, ob = out_dtype == T2H_DTYPE_BF16;
    if ((!xb && x_dtype != T2H_DTYPE_F32) || (!ob && out_dtype != T2H_DTYPE_F32)) return T2H_ERR_DTYPE;
    // fp32 rows of 1024..8192 values in whole KiB-elements, 16-byte aligned: the register-resident kernel
    const bool aligned = ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w) |
                           reinterpret_cast<uintptr_t>(out)) & 15) == 0;
    if (!xb && aligned && h % 1024 == 0 && h <= 8192) {
        const uint32_t nch = h / 1024;
        auto go = [&](auto nc) {
            constexpr int NC = decltype(nc)::value;
            const float* xf = static_cast<const float*>(x);
            if (ob)
                hipLaunchKernelGGL((rms_norm_rows_kernel<NC, true>), dim3(rows), dim3(256), 0, s, xf, w, out, h, eps);
            else
                hipLaunchKernelGGL((rms_norm_rows_kernel<NC, false>), dim3(rows), dim3(256), 0, s, xf, w, out, h, eps);
        };
        switch (nch) {
            case 1: go(std::integral_constant<int, 1>{}); break;
            case 2: go(std::integral_constant<int, 2>{}); break;
            case 3: go(std::integral_constant<int, 3>{}); break;
            case 4: go(std::integral_constant<int, 4>{}); break;
            case 5: go(std::integral_constant<int, 5>{}); break;
            case 6: go(std::integral_constant<int, 6>{}); break;
            case 7: go(std::integral_constant<int, 7>{}); break;
            default: go(std::integral_constant<int, 8>{}); break;
        }
        T2H_LAUNCH_CHECK();
        return T2H_OK;
    }
    if (xb && ob) hipLaunchKernelGGL((rms_norm_kernel<true, true>), dim3(rows), dim3(256), 0, s, x, w, out, h, eps);
    else if (xb) hipLaunchKernelGGL((rms_norm_kernel<true, false>), dim3(rows), dim3(256), 0, s, x, w, out, h, eps);
    else if (ob) hipLaunchKernelGGL((rms_norm_kernel<false, true>), dim3(rows), dim3(256), 0, s, x, w, out, h, eps);
    else hipLaunchKernelGGL((rms_norm_kernel<false, false>), dim3(rows), dim3(256), 0, s, x, w, out, h, eps);
    T2H_LAUNCH_CHECK();
    return T2H_OK;
}

extern "C" int t2h_swiglu(const void* gate, const void* up, int in_dtype, void* out, uint64_t n, void* stream) {
    if (!gate || !up || !out) return T2H_ERR_NULL;
    if (n == 0) return T2H_OK;
    const uint64_t grid = (n + 255) / 256;
    if (grid > 0x7fffffffull) return T2H_ERR_SHAPE;
    hipStream_t s = (hipStream_t)stream;
    if (in_dtype == T2H_DTYPE_BF16)
        hipLaunchKernelGGL(swiglu_kernel<true>, dim3((uint32_t)grid), dim3(256), 0, s, gate, up, (uint16_t*)out, n);
    else if (in_dtype == T2H_DTYPE_F32)
        hipLaunchKernelGGL(swiglu_kernel<false>, dim3((uint32_t)grid), dim3(256), 0, s, gate, up, (uint16_t*)out, n);
    else
        return T2H_ERR_DTYPE;
    T2H_LAUNCH_CHECK();
    return T2H_OK;
}
