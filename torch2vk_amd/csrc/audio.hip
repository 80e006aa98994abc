// Qwen3-ASR audio tower: the memory-bound ops around the encoder's GEMMs and
// attention, and the text side's Q8_0 embedding and audio injection.
//
//   im2col          conv2d front-end as (im2col -> Q8_0 GEMM with bias + GELU):
//                   CONV2D_Q8_0W_F32B_F16{,_2,_3}
//                   (src/models/quantized_qwen3_asr/shaders/conv2d_q8_0w_f32b_f16.py:114-136)
//                   and the (B, C*F, T) flatten + transpose before conv_out
//                   (pytorch_modules.py:463-466), which is the same gather with
//                   a (F x 1) kernel
//   layer_norm      LAYER_NORM_F32W_F32B_F32 (shaders/layer_norm_f32w_f32b_f32.py:77-105)
//   gelu            GELU_F32 (shaders/gelu_f32.py:61-82), when not fused into a GEMM
//   index_select    INDEX_SELECT_F32 over rows (shaders/index_select_f32_c6680f8d95.py)
//   index_copy      INDEX_COPY_F32 over rows, the audio injection
//                   (dispatch/audio_inject.py:11-13, pytorch_modules.py:16-28)
//   embedding_q8_0  EMBEDDING_Q8_0_F32 (shaders/embedding_q8_0_f32.py:90-97)
//
// All of them are HBM-bound byte movers: coalesced 4- to 16-byte accesses,
// one pass, no LDS.
#include "common.h"

namespace t2h {

// ------------------------------------------------------------- im2col --

struct Im2colArgs {
    int64_t sb, sc, sh, sw;  // input strides in elements
    uint32_t channels, in_h, in_w;
    uint32_t kh, kw, stride_h, stride_w, pad_h, pad_w;
    uint32_t out_h, out_w;
    uint32_t out_cols;       // row length of the output (>= channels * kh * kw)
    uint32_t pad_threads;    // threads per row that zero the columns past channels * kh * kw
    uint64_t rows;           // batch * out_h * out_w
    uint32_t dil_w;          // tap spacing along w (1: plain conv)
};

template <typename T>
__device__ __forceinline__ uint16_t to_bf16_bits(T v);
template <>
__device__ __forceinline__ uint16_t to_bf16_bits<float>(float v) {
    return (uint16_t)f32_to_bf16_bits(v);
}
template <>
__device__ __forceinline__ uint16_t to_bf16_bits<uint16_t>(uint16_t v) {
    return v;
}

// Thread (row, c) writes the kh * kw columns of channel c of output row
// (b, oh, ow): consecutive threads read consecutive channels of a
// channels-last input and write consecutive runs of one output row.
template <typename T>
__global__ __launch_bounds__(256) void im2col_kernel(const T* __restrict__ x, uint16_t* __restrict__ out,
                                                     const Im2colArgs a) {
    const uint64_t per_row = (uint64_t)a.channels + a.pad_threads;
    const uint64_t idx = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= a.rows * per_row) return;
    const uint64_t row = idx / per_row;
    const uint32_t c = (uint32_t)(idx - row * per_row);
    uint16_t* orow = out + row * a.out_cols;
    const uint32_t taps = a.kh * a.kw;
    if (c >= a.channels) {
        const uint32_t first = a.channels * taps + 8u * (c - a.channels);
        const uint32_t last = min(first + 8u, a.out_cols);
        for (uint32_t j = first; j < last; ++j) orow[j] = 0;
        return;
    }
    const uint32_t ow = (uint32_t)(row % a.out_w);
    const uint64_t t = row / a.out_w;
    const uint32_t oh = (uint32_t)(t % a.out_h);
    const uint64_t b = t / a.out_h;
    const T* xc = x + (int64_t)b * a.sb + (int64_t)c * a.sc;
    uint16_t* dst = orow + (uint64_t)c * taps;
    for (uint32_t fh = 0; fh < a.kh; ++fh) {
        const int ih = (int)(oh * a.stride_h + fh) - (int)a.pad_h;
        const bool h_ok = ih >= 0 && ih < (int)a.in_h;
        for (uint32_t fw = 0; fw < a.kw; ++fw) {
            const int iw = (int)(ow * a.stride_w + fw * a.dil_w) - (int)a.pad_w;
            uint16_t v = 0;
            if (h_ok && iw >= 0 && iw < (int)a.in_w) v = to_bf16_bits<T>(xc[(int64_t)ih * a.sh + (int64_t)iw * a.sw]);
            dst[fh * a.kw + fw] = v;
        }
    }
}

// --------------------------------------------------------- layer norm --

template <typename T>
__device__ __forceinline__ float4 load4(const T* p);
template <>
__device__ __forceinline__ float4 load4<float>(const float* p) {
    return *reinterpret_cast<const float4*>(p);
}
template <>
__device__ __forceinline__ float4 load4<uint16_t>(const uint16_t* p) {
    const uint2 u = *reinterpret_cast<const uint2*>(p);
    return make_float4(bf16_bits_to_f32(u.x & 0xffffu), bf16_bits_to_f32(u.x >> 16), bf16_bits_to_f32(u.y & 0xffffu),
                       bf16_bits_to_f32(u.y >> 16));
}

template <typename T>
__device__ __forceinline__ void store4(T* p, float4 v);
template <>
__device__ __forceinline__ void store4<float>(float* p, float4 v) {
    *reinterpret_cast<float4*>(p) = v;
}
template <>
__device__ __forceinline__ void store4<uint16_t>(uint16_t* p, float4 v) {
    *reinterpret_cast<uint2*>(p) = make_uint2(pack_bf16x2(v.x, v.y), pack_bf16x2(v.z, v.w));
}

// One wave per row, 4 consecutive values per lane per step; mean, then the
// sum of squared deviations (two passes over the row, the second from cache).
template <typename TI, typename TO>
__global__ __launch_bounds__(256) void layer_norm_kernel(const TI* __restrict__ x, const float* __restrict__ w,
                                                         const float* __restrict__ bias, TO* __restrict__ out,
                                                         uint32_t rows, uint32_t cols, float eps) {
    const uint32_t row = blockIdx.x * 4 + (threadIdx.x >> 6);
    const uint32_t lane = threadIdx.x & 63;
    if (row >= rows) return;
    const TI* xr = x + (size_t)row * cols;
    float s = 0.0f;
    for (uint32_t c = 4 * lane; c < cols; c += 256) {
        const float4 v = load4<TI>(xr + c);
        s += (v.x + v.y) + (v.z + v.w);
    }
    const float mean = wave_sum(s) / (float)cols;
    float q = 0.0f;
    for (uint32_t c = 4 * lane; c < cols; c += 256) {
        const float4 v = load4<TI>(xr + c);
        const float a = v.x - mean, b = v.y - mean, cc = v.z - mean, d = v.w - mean;
        q += (a * a + b * b) + (cc * cc + d * d);
    }
    const float inv = rsqrtf(wave_sum(q) / (float)cols + eps);
    TO* orow = out + (size_t)row * cols;
    for (uint32_t c = 4 * lane; c < cols; c += 256) {
        const float4 v = load4<TI>(xr + c);
        const float4 g = *reinterpret_cast<const float4*>(w + c);
        const float4 bb = *reinterpret_cast<const float4*>(bias + c);
        store4<TO>(orow + c, make_float4(fmaf((v.x - mean) * inv, g.x, bb.x), fmaf((v.y - mean) * inv, g.y, bb.y),
                                         fmaf((v.z - mean) * inv, g.z, bb.z), fmaf((v.w - mean) * inv, g.w, bb.w)));
    }
}

// --------------------------------------------------------------- gelu --

__device__ __forceinline__ float gelu_erf_f(float v) { return gelu_as(v); }  // erf by Abramowitz-Stegun 7.1.26

template <typename TI, typename TO>
__global__ __launch_bounds__(256) void gelu_kernel(const TI* __restrict__ x, TO* __restrict__ out, uint64_t n4) {
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n4) return;
    const float4 v = load4<TI>(x + 4 * i);
    store4<TO>(out + 4 * i, make_float4(gelu_erf_f(v.x), gelu_erf_f(v.y), gelu_erf_f(v.z), gelu_erf_f(v.w)));
}

// ------------------------------------------------------- row gathers --

// out[i] = src[idx[i]] (4-byte words; a row index out of range gives zeros)
__global__ __launch_bounds__(256) void index_select_rows_kernel(const uint32_t* __restrict__ src, uint64_t src_rows,
                                                                uint32_t row_words, const int64_t* __restrict__ idx,
                                                                uint32_t n, uint32_t* __restrict__ out) {
    const uint64_t t = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= (uint64_t)n * row_words) return;
    const uint64_t i = t / row_words;
    const uint32_t j = (uint32_t)(t - i * row_words);
    const int64_t r = idx[i];
    out[t] = (r >= 0 && (uint64_t)r < src_rows) ? src[(uint64_t)r * row_words + j] : 0u;
}

// dst[idx[i]] = src[i] (4-byte words; a row index out of range is skipped)
__global__ __launch_bounds__(256) void index_copy_rows_kernel(uint32_t* __restrict__ dst, uint64_t dst_rows,
                                                              uint32_t row_words, const int64_t* __restrict__ idx,
                                                              uint32_t n, const uint32_t* __restrict__ src) {
    const uint64_t t = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= (uint64_t)n * row_words) return;
    const uint64_t i = t / row_words;
    const uint32_t j = (uint32_t)(t - i * row_words);
    const int64_t r = idx[i];
    if (r >= 0 && (uint64_t)r < dst_rows) dst[(uint64_t)r * row_words + j] = src[t];
}

// ---------------------------------------------------- Q8_0 embedding --

// Thread (token, block) dequantises one 34-byte Q8_0 block: d (fp16) * int8.
__global__ __launch_bounds__(256) void embedding_q8_0_kernel(const uint8_t* __restrict__ w, uint64_t vocab,
                                                             const int64_t* __restrict__ ids, uint32_t n_ids,
                                                             uint32_t dim, float* __restrict__ out) {
    const uint32_t blocks = dim / 32;
    const uint64_t t = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= (uint64_t)n_ids * blocks) return;
    const uint64_t i = t / blocks;
    const uint32_t blk = (uint32_t)(t - i * blocks);
    float* o = out + i * dim + 32 * blk;
    const int64_t id = ids[i];
    if (id < 0 || (uint64_t)id >= vocab) {
        for (int j = 0; j < 32; j += 4) *reinterpret_cast<float4*>(o + j) = make_float4(0.f, 0.f, 0.f, 0.f);
        return;
    }
    const uint8_t* p = w + (uint64_t)id * blocks * 34 + (uint64_t)blk * 34;
    const uint16_t* h = reinterpret_cast<const uint16_t*>(p);  // blocks are 2-byte aligned
    const float d = f16_bits_to_f32(h[0]);
#pragma unroll
    for (int j = 0; j < 16; j += 2) {
        const uint32_t q01 = h[1 + j], q23 = h[2 + j];
        *reinterpret_cast<float4*>(o + 2 * j) =
            make_float4(d * (float)(int8_t)(q01 & 0xffu), d * (float)(int8_t)(q01 >> 8),
                        d * (float)(int8_t)(q23 & 0xffu), d * (float)(int8_t)(q23 >> 8));
    }
}

static inline uint32_t grid_for(uint64_t threads) { return (uint32_t)((threads + 255) / 256); }

}  // namespace t2h

using namespace t2h;

extern "C" int t2h_im2col(const void* x, int x_dtype, const int64_t* x_strides, uint32_t batch, uint32_t channels,
                          uint32_t in_h, uint32_t in_w, uint32_t kh, uint32_t kw, uint32_t stride_h,
                          uint32_t stride_w, uint32_t pad_h, uint32_t pad_w, uint32_t out_h, uint32_t out_w,
                          void* out, uint32_t out_cols, void* stream) {
    if (!x || !x_strides || !out) return T2H_ERR_NULL;
    if (x_dtype != T2H_DTYPE_F32 && x_dtype != T2H_DTYPE_BF16) return T2H_ERR_DTYPE;
    if (kh == 0 || kw == 0 || stride_h == 0 || stride_w == 0 || channels == 0) return T2H_ERR_SHAPE;
    if ((uint64_t)channels * kh * kw > out_cols) return T2H_ERR_SHAPE;
    // every output position's receptive field starts inside the padded input
    if (out_h > 0 && (uint64_t)(out_h - 1) * stride_h > (uint64_t)in_h + 2 * pad_h) return T2H_ERR_SHAPE;
    if (out_w > 0 && (uint64_t)(out_w - 1) * stride_w > (uint64_t)in_w + 2 * pad_w) return T2H_ERR_SHAPE;
    if (in_h > 0x7fffffffu || in_w > 0x7fffffffu || pad_h > 0xffffu || pad_w > 0xffffu) return T2H_ERR_SHAPE;
    for (int i = 0; i < 4; ++i)
        if (x_strides[i] < 0) return T2H_ERR_ARG;
    Im2colArgs a;
    a.sb = x_strides[0];
    a.sc = x_strides[1];
    a.sh = x_strides[2];
    a.sw = x_strides[3];
    a.channels = channels;
    a.in_h = in_h;
    a.in_w = in_w;
    a.kh = kh;
    a.kw = kw;
    a.stride_h = stride_h;
    a.stride_w = stride_w;
    a.pad_h = pad_h;
    a.pad_w = pad_w;
    a.dil_w = 1;
    a.out_h = out_h;
    a.out_w = out_w;
    a.out_cols = out_cols;
    a.pad_threads = (out_cols - channels * kh * kw + 7) / 8;
    a.rows = (uint64_t)batch * out_h * out_w;
    const uint64_t threads = a.rows * ((uint64_t)channels + a.pad_threads);
    if (threads == 0) return T2H_OK;
    if (threads / 256 >= 0x7fffffffu) return T2H_ERR_SHAPE;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    uint16_t* o = reinterpret_cast<uint16_t*>(out);
    if (x_dtype == T2H_DTYPE_F32)
        hipLaunchKernelGGL(im2col_kernel<float>, dim3(grid_for(threads)), dim3(256), 0, s,
                           reinterpret_cast<const float*>(x), o, a);
    else
        hipLaunchKernelGGL(im2col_kernel<uint16_t>, dim3(grid_for(threads)), dim3(256), 0, s,
                           reinterpret_cast<const uint16_t*>(x), o, a);
    T2H_LAUNCH_CHECK();
    return T2H_OK;
}

extern "C" int t2h_layer_norm(const void* x, int x_dtype, const float* w, const float* b, void* out, int out_dtype,
                              uint32_t rows, uint32_t cols, float eps, void* stream) {
    if (!x || !w || !b || !out) return T2H_ERR_NULL;
    if ((x_dtype != T2H_DTYPE_F32 && x_dtype != T2H_DTYPE_BF16) ||
        (out_dtype != T2H_DTYPE_F32 && out_dtype != T2H_DTYPE_BF16))
        return T2H_ERR_DTYPE;
    if (cols == 0 || cols % 4 != 0) return T2H_ERR_SHAPE;
    const uintptr_t bits = reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(out) |
                           reinterpret_cast<uintptr_t>(w) | reinterpret_cast<uintptr_t>(b);
    if ((bits & 15) != 0) return T2H_ERR_ALIGN;
    if (rows == 0) return T2H_OK;
    const dim3 grid((rows + 3) / 4), block(256);
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    if (x_dtype == T2H_DTYPE_F32) {
        const float* xi = reinterpret_cast<const float*>(x);
        if (out_dtype == T2H_DTYPE_BF16)
            hipLaunchKernelGGL((layer_norm_kernel<float, uint16_t>), grid, block, 0, s, xi, w, b,
                               reinterpret_cast<uint16_t*>(out), rows, cols, eps);
        else
            hipLaunchKernelGGL((layer_norm_kernel<float, float>), grid, block, 0, s, xi, w, b,
                               reinterpret_cast<float*>(out), rows, cols, eps);
    } else {
        const uint16_t* xi = reinterpret_cast<const uint16_t*>(x);
        if (out_dtype == T2H_DTYPE_BF16)
            hipLaunchKernelGGL((layer_norm_kernel<uint16_t, uint16_t>), grid, block, 0, s, xi, w, b,
                               reinterpret_cast<uint16_t*>(out), rows, cols, eps);
        else
            hipLaunchKernelGGL((layer_norm_kernel<uint16_t, float>), grid, block, 0, s, xi, w, b,
                               reinterpret_cast<float*>(out), rows, cols, eps);
    }
    T2H_LAUNCH_CHECK();
    return T2H_OK;
}

extern "C" int t2h_gelu(const void* x, int x_dtype, void* out, int out_dtype, uint64_t n, void* stream) {
    if (!x || !out) return T2H_ERR_NULL;
    if ((x_dtype != T2H_DTYPE_F32 && x_dtype != T2H_DTYPE_BF16) ||
        (out_dtype != T2H_DTYPE_F32 && out_dtype != T2H_DTYPE_BF16))
        return T2H_ERR_DTYPE;
    if (n % 4 != 0) return T2H_ERR_SHAPE;
    const uintptr_t bits = reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(out);
    if ((bits & 7) != 0) return T2H_ERR_ALIGN;
    if (n == 0) return T2H_OK;
    const uint64_t n4 = n / 4;
    if (n4 / 256 >= 0x7fffffffu) return T2H_ERR_SHAPE;
    const dim3 grid(grid_for(n4)), block(256);
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    if (x_dtype == T2H_DTYPE_F32) {
        const float* xi = reinterpret_cast<const float*>(x);
        if (out_dtype == T2H_DTYPE_BF16)
            hipLaunchKernelGGL((gelu_kernel<float, uint16_t>), grid, block, 0, s, xi, reinterpret_cast<uint16_t*>(out), n4);
        else
            hipLaunchKernelGGL((gelu_kernel<float, float>), grid, block, 0, s, xi, reinterpret_cast<float*>(out), n4);
    } else {
        const uint16_t* xi = reinterpret_cast<const uint16_t*>(x);
        if (out_dtype == T2H_DTYPE_BF16)
            hipLaunchKernelGGL((gelu_kernel<uint16_t, uint16_t>), grid, block, 0, s, xi,
                               reinterpret_cast<uint16_t*>(out), n4);
        else
            hipLaunchKernelGGL((gelu_kernel<uint16_t, float>), grid, block, 0, s, xi, reinterpret_cast<float*>(out), n4);
    }
    T2H_LAUNCH_CHECK();
    return T2H_OK;
}

extern "C" int t2h_index_select_rows(const void* src, uint64_t src_rows, uint32_t row_bytes, const int64_t* idx,
                                     uint32_t n, void* out, void* stream) {
    if (!src || !idx || !out) return T2H_ERR_NULL;
    if (row_bytes == 0 || row_bytes % 4 != 0) return T2H_ERR_SHAPE;
    if (((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(out)) & 3) != 0) return T2H_ERR_ALIGN;
    const uint64_t threads = (uint64_t)n * (row_bytes / 4);
    if (threads == 0) return T2H_OK;
    if (threads / 256 >= 0x7fffffffu) return T2H_ERR_SHAPE;
    hipLaunchKernelGGL(index_select_rows_kernel, dim3(grid_for(threads)), dim3(256), 0,
                       reinterpret_cast<hipStream_t>(stream), reinterpret_cast<const uint32_t*>(src), src_rows,
                       row_bytes / 4, idx, n, reinterpret_cast<uint32_t*>(out));
    T2H_LAUNCH_CHECK();
    return T2H_OK;
}

extern "C" int t2h_index_copy_rows(void* dst, uint64_t dst_rows, uint32_t row_bytes, const int64_t* idx, uint32_t n,
                                   const void* src, void* stream) {
    if (!dst || !idx || !src) return T2H_ERR_NULL;
    if (row_bytes == 0 || row_bytes % 4 != 0) return T2H_ERR_SHAPE;
    if (((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) & 3) != 0) return T2H_ERR_ALIGN;
    const uint64_t threads = (uint64_t)n * (row_bytes / 4);
    if (threads == 0) return T2H_OK;
    if (threads / 256 >= 0x7fffffffu) return T2H_ERR_SHAPE;
    hipLaunchKernelGGL(index_copy_rows_kernel, dim3(grid_for(threads)), dim3(256), 0,
                       reinterpret_cast<hipStream_t>(stream), reinterpret_cast<uint32_t*>(dst), dst_rows,
                       row_bytes / 4, idx, n, reinterpret_cast<const uint32_t*>(src));
    T2H_LAUNCH_CHECK();
    return T2H_OK;
}

extern "C" int t2h_embedding_q8_0(const void* w, uint64_t vocab, const int64_t* ids, uint32_t n_ids, uint32_t dim,
                                  float* out, void* stream) {
    if (!w || !ids || !out) return T2H_ERR_NULL;
    if (dim == 0 || dim % 32 != 0) return T2H_ERR_SHAPE;
    if ((reinterpret_cast<uintptr_t>(w) & 1) != 0 || (reinterpret_cast<uintptr_t>(out) & 15) != 0)
        return T2H_ERR_ALIGN;
    const uint64_t threads = (uint64_t)n_ids * (dim / 32);
    if (threads == 0) return T2H_OK;
    if (threads / 256 >= 0x7fffffffu) return T2H_ERR_SHAPE;
    hipLaunchKernelGGL(embedding_q8_0_kernel, dim3(grid_for(threads)), dim3(256), 0,
                       reinterpret_cast<hipStream_t>(stream), reinterpret_cast<const uint8_t*>(w), vocab, ids, n_ids,
                       dim, out);
    T2H_LAUNCH_CHECK();
    return T2H_OK;
}

// conv1d taps of x [B, C, L] (any strides): row b * out_len + t holds
// x[b, c, t * stride + k * dilation - pad] at column c * K + k (zero outside
// the input), the reference conv1d's operand order
// (src/models/quantized_omnivoice/shaders/conv1d_q8_0w_f32b_f32.py, conv_input_value);
// columns past C * K are zero.  The 2-D kernel with one row.
extern "C" int t2h_im2col_1d(const void* x, int x_dtype, const int64_t* x_strides, uint32_t batch, uint32_t channels,
                             uint32_t length, uint32_t k, uint32_t stride, uint32_t pad, uint32_t dilation,
                             uint32_t out_len, void* out, uint32_t out_cols, void* stream) {
    if (!x || !x_strides || !out) return T2H_ERR_NULL;
    if (x_dtype != T2H_DTYPE_F32 && x_dtype != T2H_DTYPE_BF16) return T2H_ERR_DTYPE;
    if (k == 0 || stride == 0 || dilation == 0 || channels == 0) return T2H_ERR_SHAPE;
    if ((uint64_t)channels * k > out_cols) return T2H_ERR_SHAPE;
    if (out_len > 0 && (uint64_t)(out_len - 1) * stride > (uint64_t)length + 2 * pad) return T2H_ERR_SHAPE;
    if (length > 0x7fffffffu || pad > 0xffffu || (uint64_t)(k - 1) * dilation > 0x7fffffffu) return T2H_ERR_SHAPE;
    for (int i = 0; i < 3; ++i)
        if (x_strides[i] < 0) return T2H_ERR_ARG;
    Im2colArgs a;
    a.sb = x_strides[0];
    a.sc = x_strides[1];
    a.sh = 0;
    a.sw = x_strides[2];
    a.channels = channels;
    a.in_h = 1;
    a.in_w = length;
    a.kh = 1;
    a.kw = k;
    a.stride_h = 1;
    a.stride_w = stride;
    a.pad_h = 0;
    a.pad_w = pad;
    a.dil_w = dilation;
    a.out_h = 1;
    a.out_w = out_len;
    a.out_cols = out_cols;
    a.pad_threads = (out_cols - channels * k + 7) / 8;
    a.rows = (uint64_t)batch * out_len;
    const uint64_t threads = a.rows * ((uint64_t)channels + a.pad_threads);
    if (threads == 0) return T2H_OK;
    if (threads / 256 >= 0x7fffffffu) return T2H_ERR_SHAPE;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    uint16_t* o = reinterpret_cast<uint16_t*>(out);
    if (x_dtype == T2H_DTYPE_F32)
        hipLaunchKernelGGL(im2col_kernel<float>, dim3(grid_for(threads)), dim3(256), 0, s,
                           reinterpret_cast<const float*>(x), o, a);
    else
        hipLaunchKernelGGL(im2col_kernel<uint16_t>, dim3(grid_for(threads)), dim3(256), 0, s,
                           reinterpret_cast<const uint16_t*>(x), o, a);
    T2H_LAUNCH_CHECK();
    return T2H_OK;
}

// ----------------------------------------------------------------- snake --

// y = x + sin(alpha_c x)^2 / (alpha_c + eps) per channel c of channels-last
// rows [rows, C]: the snake activation of the audio decoder, built in the
// reference from ADD_SCALAR (eps 1e-9), RECIPROCAL, MUL_BROADCAST, SIN and
// POW_SCALAR (src/models/quantized_omnivoice/dispatch/audio_decode.py:151-161).
__global__ __launch_bounds__(256) void snake_kernel(const float* __restrict__ x, const float* __restrict__ alpha,
                                                    float* __restrict__ y, uint64_t n, uint32_t channels, float eps) {
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float a = alpha[i % channels];
    const float v = x[i];
    const float s = sinf(a * v);
    y[i] = v + (1.0f / (a + eps)) * (s * s);
}

extern "C" int t2h_snake(const float* x, const float* alpha, float* out, uint64_t rows, uint32_t channels, float eps,
                         void* stream) {
    if (!x || !alpha || !out) return T2H_ERR_NULL;
    if (channels == 0) return T2H_ERR_SHAPE;
    const uint64_t n = rows * channels;
    if (n == 0) return T2H_OK;
    if (n / 256 >= 0x7fffffffu) return T2H_ERR_SHAPE;
    hipLaunchKernelGGL(snake_kernel, dim3(grid_for(n)), dim3(256), 0, reinterpret_cast<hipStream_t>(stream), x, alpha,
                       out, n, channels, eps);
    T2H_LAUNCH_CHECK();
    return T2H_OK;
}

// ------------------------------------------------------ conv transpose --

// y[b, t, co] = bias[co] + sum_ci sum_k W[ci, co K + k] x[b, ci, i] over the
// taps k with t + pad - k = i * stride, 0 <= i < L_in: CONV_TRANSPOSE1D_Q8_0W_F32B_F32
// (src/models/quantized_omnivoice/shaders/conv_transpose1d_q8_0w_f32b_f32.py:
// deconv_input_value, deconv_weight_value), reading the reference's Q8_0 rows
// [Ci, Co K] (34-byte blocks: fp16 scale + 32 int8) as they are, in fp32.
// One thread per output (b, t, co); consecutive threads take consecutive co,
// so a wave shares every x value it reads.
struct ConvTArgs {
    const float* x;
    int64_t sb, sc, sl;     // x strides (elements): batch, channel, position
    const uint8_t* w;
    const float* bias;
    float* out;             // [B, L_out, Co] contiguous
    uint32_t ci, li, co, kh, stride, pad, lo;
    uint32_t row_bytes;     // Q8_0 bytes per weight row (ceil(Co K / 32) * 34)
    uint64_t n;             // B * L_out * Co
};

__global__ __launch_bounds__(256) void conv_transpose1d_q8_0_kernel(const ConvTArgs a) {
    const uint64_t idx = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= a.n) return;
    const uint32_t co = (uint32_t)(idx % a.co);
    const uint64_t r = idx / a.co;
    const uint32_t t = (uint32_t)(r % a.lo);
    const uint64_t b = r / a.lo;
    // first tap whose input position is a whole step: (t + pad - k) % stride == 0
    const uint32_t k0 = (t + a.pad) % a.stride;
    float acc = a.bias ? a.bias[co] : 0.0f;
    for (uint32_t k = k0; k < a.kh; k += a.stride) {
        const int num = (int)t + (int)a.pad - (int)k;
        if (num < 0) break;  // k only grows
        const uint32_t i = (uint32_t)num / a.stride;
        if (i >= a.li) continue;
        const uint32_t e = co * a.kh + k;          // element of every weight row
        const uint32_t blk = e >> 5, q = e & 31u;
        const float* xi = a.x + (int64_t)b * a.sb + (int64_t)i * a.sl;
        const uint8_t* wb = a.w + (size_t)blk * 34;
        for (uint32_t c = 0; c < a.ci; ++c) {
            const uint8_t* row = wb + (size_t)c * a.row_bytes;
            const float d = f16_bits_to_f32((uint32_t)row[0] | ((uint32_t)row[1] << 8));
            const float wv = d * (float)(int8_t)row[2 + q];
            acc = fmaf(wv, xi[(int64_t)c * a.sc], acc);
        }
    }
    a.out[idx] = acc;
}

extern "C" int t2h_conv_transpose1d_q8_0(const float* x, const int64_t* x_strides, const void* w, const float* bias,
                                         float* out, uint32_t batch, uint32_t ci, uint32_t li, uint32_t co,
                                         uint32_t kh, uint32_t stride, uint32_t pad, uint32_t lo, void* stream) {
    if (!x || !x_strides || !w || !out) return T2H_ERR_NULL;
    if (ci == 0 || co == 0 || kh == 0 || stride == 0 || li == 0) return T2H_ERR_SHAPE;
    // L_out of a transposed conv plus an output padding in [0, stride): the extra last positions take the taps
    // that reach them (the reference's blocks produce stride * L_in outputs, output padding stride % 2)
    const int64_t lo_min = ((int64_t)li - 1) * stride - 2 * (int64_t)pad + kh;
    if ((int64_t)lo < lo_min || (int64_t)lo >= lo_min + stride) return T2H_ERR_SHAPE;
    if ((uint64_t)co * kh > 0x7fffffffu || pad > 0xffffu || li > 0x7fffffffu) return T2H_ERR_SHAPE;
    if (reinterpret_cast<uintptr_t>(w) % 2 != 0) return T2H_ERR_ALIGN;
    for (int i = 0; i < 3; ++i)
        if (x_strides[i] < 0) return T2H_ERR_ARG;
    ConvTArgs a;
    a.x = x;
    a.sb = x_strides[0];
    a.sc = x_strides[1];
    a.sl = x_strides[2];
    a.w = reinterpret_cast<const uint8_t*>(w);
    a.bias = bias;
    a.out = out;
    a.ci = ci;
    a.li = li;
    a.co = co;
    a.kh = kh;
    a.stride = stride;
    a.pad = pad;
    a.lo = lo;
    a.row_bytes = (uint32_t)(((uint64_t)co * kh + 31) / 32 * 34);
    a.n = (uint64_t)batch * lo * co;
    if (a.n == 0) return T2H_OK;
    if (a.n / 256 >= 0x7fffffffu) return T2H_ERR_SHAPE;
    hipLaunchKernelGGL(conv_transpose1d_q8_0_kernel, dim3(grid_for(a.n)), dim3(256), 0,
                       reinterpret_cast<hipStream_t>(stream), a);
    T2H_LAUNCH_CHECK();
    return T2H_OK;
}
