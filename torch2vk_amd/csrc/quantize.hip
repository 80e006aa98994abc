// GGUF block quantizers and dequantizers on gfx950.
//
// Replaces GGUF_QUANTIZE_{Q8_0,Q4_K,Q6_K}_F32 (src/torch2vk/quantize/vulkan.py:91-636)
// and their host wrappers quantize_*_vulkan (vulkan.py:25-66).  The fp32
// operation order follows the GLSL line by line; a*b+c is never contracted
// (this file is built with -ffp-contract=off and the pragma below), division
// and sqrt are the correctly rounded IEEE operations, fp16 rounding is RNE and
// GLSL round() ties go to even.  The result is bit-identical to the CPU
// restatement used as the test oracle.
//
// Parallel layout: one lane per 32-value Q4_K sub-block (8 lanes per
// superblock), one lane per 16-value Q6_K sub-block (16 lanes per
// superblock), one lane per Q8_0 value (32 lanes per block).
#include "common.h"

#pragma clang fp contract(off)

namespace t2h {

__device__ __forceinline__ float round_f16(float v) { return f16_bits_to_f32(f32_to_f16_bits_rne(v)); }
__device__ __forceinline__ float clampf_(float x, float lo, float hi) { return fminf(fmaxf(x, lo), hi); }

// ------------------------------------------------------------------ Q8_0 --

__device__ __forceinline__ float round_away(float value) {
    const float absolute = fabsf(value);
    const float floored = floorf(absolute);
    const float rounded = floored + floorf(2.0f * (absolute - floored));
    const float s = value > 0.0f ? 1.0f : (value < 0.0f ? -1.0f : 0.0f);
    return s * rounded;
}

// block = 64 threads = two Q8_0 blocks; grid.x over (rows * blocks_per_row / 2)
__global__ __launch_bounds__(64) void quantize_q8_0_kernel(const float* __restrict__ x, uint8_t* __restrict__ out,
                                                           uint32_t k, uint64_t total_blocks) {
    const uint64_t blk = (uint64_t)blockIdx.x * 2 + (threadIdx.x >> 5);
    const int lane = threadIdx.x & 31;
    if (blk >= total_blocks) return;
    const uint32_t bpr = k / 32;
    const uint64_t row = blk / bpr;
    const uint64_t b = blk % bpr;
    const float value = x[row * k + b * 32 + lane];
    float amax = 0.0f;
    // sequential max in index order, as the reference's lane 0 does
    for (int i = 0; i < 32; ++i) {
        const float vi = __shfl(value, (threadIdx.x & 32) + i, 64);
        amax = fmaxf(amax, fabsf(vi));
    }
    const float block_scale = amax / 127.0f;
    const float inv_scale = block_scale == 0.0f ? 0.0f : 1.0f / block_scale;
    int quant = (int)round_away(value * inv_scale);
    quant = quant < -128 ? -128 : (quant > 127 ? 127 : quant);
    uint8_t* o = out + blk * 34;
    if (lane == 0) {
        const uint32_t d16 = f32_to_f16_bits_rne(block_scale);
        o[0] = (uint8_t)(d16 & 0xffu);
        o[1] = (uint8_t)(d16 >> 8);
    }
    o[2 + lane] = (uint8_t)(quant & 255);
}

// ------------------------------------------------------------------ Q4_K --

__device__ __forceinline__ uint32_t rounded_code(float value, uint32_t max_code) {
    return (uint32_t)clampf_(floorf(value + 0.5f), 0.0f, (float)max_code);
}

__device__ float weighted_quant_error(const float* v, float scale, float minimum, float inv_scale) {
    float error = 0.0f;
    float sum_x2 = 0.0f;
    for (int i = 0; i < 32; ++i) {
        const float t = v[i] * v[i];
        sum_x2 = sum_x2 + t;
    }
    const float av_x = sqrtf(sum_x2 / 32.0f);
    for (int i = 0; i < 32; ++i) {
        const float weight = av_x + fabsf(v[i]);
        const float level = (float)rounded_code(inv_scale * (v[i] - minimum), 15u);
        const float sl = scale * level;
        const float diff = (sl + minimum) - v[i];
        const float wd = weight * diff;
        error = error + wd * diff;
    }
    return error;
}

__device__ float choose_subblock_scale(const float* v, float* min_offset) {
    float min_value = v[0];
    float max_value = v[0];
    float sum_x2 = 0.0f;
    for (int i = 0; i < 32; ++i) {
        min_value = fminf(min_value, v[i]);
        max_value = fmaxf(max_value, v[i]);
        const float t = v[i] * v[i];
        sum_x2 = sum_x2 + t;
    }
    if (min_value > 0.0f) min_value = 0.0f;
    if (max_value == min_value) {
        *min_offset = -min_value;
        return 0.0f;
    }
    const float av_x = sqrtf(sum_x2 / 32.0f);
    float sum_w = 0.0f;
    float sum_x = 0.0f;
    for (int i = 0; i < 32; ++i) {
        const float weight = av_x + fabsf(v[i]);
        sum_w = sum_w + weight;
        const float wx = weight * v[i];
        sum_x = sum_x + wx;
    }
    float inv_scale = 15.0f / (max_value - min_value);
    float best_scale = 1.0f / inv_scale;
    float best_min = min_value;
    float best_error = weighted_quant_error(v, best_scale, best_min, inv_scale);
    for (uint32_t step = 0; step <= 20u; ++step) {
        const float stepped = 0.1f * (float)step;
        inv_scale = (14.0f + stepped) / (max_value - min_value);
        float sum_l = 0.0f, sum_l2 = 0.0f, sum_xl = 0.0f;
        for (int i = 0; i < 32; ++i) {
            const float weight = av_x + fabsf(v[i]);
            const float level = (float)rounded_code(inv_scale * (v[i] - min_value), 15u);
            const float wl = weight * level;
            sum_l = sum_l + wl;
            const float wll = wl * level;
            sum_l2 = sum_l2 + wll;
            const float wlx = wl * v[i];
            sum_xl = sum_xl + wlx;
        }
        const float det_a = sum_w * sum_l2;
        const float det_b = sum_l * sum_l;
        const float determinant = det_a - det_b;
        if (determinant > 0.0f) {
            const float sa = sum_w * sum_xl;
            const float sb = sum_x * sum_l;
            float candidate_scale = (sa - sb) / determinant;
            const float ma = sum_l2 * sum_x;
            const float mb = sum_l * sum_xl;
            float candidate_min = (ma - mb) / determinant;
            if (candidate_min > 0.0f) {
                candidate_min = 0.0f;
                candidate_scale = sum_l2 > 0.0f ? sum_xl / sum_l2 : 0.0f;
            }
            const float candidate_error = weighted_quant_error(v, candidate_scale, candidate_min, inv_scale);
            if (candidate_error < best_error) {
                best_error = candidate_error;
                best_scale = candidate_scale;
                best_min = candidate_min;
            }
        }
    }
    *min_offset = fmaxf(0.0f, -best_min);
    return fmaxf(0.0f, best_scale);
}

// block = 64 threads = 8 superblocks, 8 lanes (one sub-block each) per superblock
__global__ __launch_bounds__(64) void quantize_q4_k_kernel(const float* __restrict__ x, uint8_t* __restrict__ out,
                                                           uint32_t k, uint64_t total_blocks) {
    const uint64_t blk = (uint64_t)blockIdx.x * 8 + (threadIdx.x >> 3);
    const int sub = threadIdx.x & 7;
    const int group_base = threadIdx.x & ~7;
    if (blk >= total_blocks) return;
    const uint32_t bpr = k / 256;
    const uint64_t row = blk / bpr;
    const uint64_t b = blk % bpr;
    const float* src = x + row * k + b * 256 + sub * 32;
    float v[32];
    for (int i = 0; i < 32; ++i) v[i] = src[i];

    float min_offset = 0.0f;
    const float sscale = choose_subblock_scale(v, &min_offset);

    // lane 0 of the superblock's semantics: sequential max over sub-blocks 0..7
    float max_scale = 0.0f, max_min = 0.0f;
    float scales[8], mins[8];
    for (int j = 0; j < 8; ++j) {
        scales[j] = __shfl(sscale, group_base + j, 64);
        mins[j] = __shfl(min_offset, group_base + j, 64);
        max_scale = fmaxf(max_scale, scales[j]);
        max_min = fmaxf(max_min, mins[j]);
    }
    float d_scale = max_scale > 0.0f ? max_scale / 63.0f : 0.0f;
    float d_min = max_min > 0.0f ? max_min / 63.0f : 0.0f;
    const float inv_scale = max_scale > 0.0f ? 63.0f / max_scale : 0.0f;
    const float inv_min = max_min > 0.0f ? 63.0f / max_min : 0.0f;
    uint32_t scale_codes[8], min_codes[8];
    for (int j = 0; j < 8; ++j) {
        scale_codes[j] = rounded_code(scales[j] * inv_scale, 63u);
        min_codes[j] = rounded_code(mins[j] * inv_min, 63u);
    }
    d_scale = round_f16(d_scale);
    d_min = round_f16(d_min);

    const float scale = d_scale * (float)scale_codes[sub];
    const float minimum = d_min * (float)min_codes[sub];
    uint32_t quants[32];
    for (int i = 0; i < 32; ++i) {
        uint32_t q = 0u;
        if (scale > 0.0f) q = rounded_code((v[i] + minimum) / scale, 15u);
        quants[i] = q;
    }
    uint8_t* o = out + blk * 144;
    if (sub == 0) {
        const uint32_t d16 = f32_to_f16_bits_rne(d_scale);
        const uint32_t m16 = f32_to_f16_bits_rne(d_min);
        o[0] = (uint8_t)(d16 & 0xffu);
        o[1] = (uint8_t)(d16 >> 8);
        o[2] = (uint8_t)(m16 & 0xffu);
        o[3] = (uint8_t)(m16 >> 8);
        for (int i = 0; i < 4; ++i) {
            o[4 + i] = (uint8_t)((scale_codes[i] & 63u) | ((scale_codes[i + 4] & 48u) << 2));
            o[8 + i] = (uint8_t)((min_codes[i] & 63u) | ((min_codes[i + 4] & 48u) << 2));
            o[12 + i] = (uint8_t)((scale_codes[i + 4] & 15u) | ((min_codes[i + 4] & 15u) << 4));
        }
    }
    // sub-block s lives in nibble group s/2: low nibbles if s even, high if odd
    const int group = sub >> 1;
    const bool high = (sub & 1) != 0;
    // combine with the partner lane's nibbles so each byte is written once
    for (int i = 0; i < 32; ++i) {
        const uint32_t partner = (uint32_t)__shfl((int)quants[i], threadIdx.x ^ 1, 64);
        if (!high) o[16 + group * 32 + i] = (uint8_t)((quants[i] & 15u) | ((partner & 15u) << 4));
    }
}

// ------------------------------------------------------------------ Q6_K --

__device__ __forceinline__ int nearest_int(float value) { return (int)rintf(value); }
__device__ __forceinline__ int clampi(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }

__device__ float make_qx_quants16(const float* v, int* levels) {
    float max_value = 0.0f, max_abs = 0.0f;
    for (int i = 0; i < 16; ++i) {
        const float a = fabsf(v[i]);
        if (a > max_abs) {
            max_abs = a;
            max_value = v[i];
        }
    }
    if (max_abs < 1.0e-12f) {
        for (int i = 0; i < 16; ++i) levels[i] = 32;
        return 0.0f;
    }
    float inv_scale = -32.0f / max_value;
    float sum_lx = 0.0f, sum_l2 = 0.0f;
    for (int i = 0; i < 16; ++i) {
        const int level = clampi(nearest_int(inv_scale * v[i]), -32, 31);
        levels[i] = level + 32;
        const float weight = v[i] * v[i];
        const float wv = weight * v[i];
        const float wvl = wv * (float)level;
        sum_lx = sum_lx + wvl;
        const float wll = weight * (float)(level * level);
        sum_l2 = sum_l2 + wll;
    }
    float scale = sum_l2 > 0.0f ? sum_lx / sum_l2 : 0.0f;
    float best = scale * sum_lx;
    for (int step = -9; step <= 9; ++step) {
        if (step == 0) continue;
        const float stepped = 0.1f * (float)step;
        const float numer = 32.0f + stepped;
        inv_scale = -numer / max_value;
        sum_lx = 0.0f;
        sum_l2 = 0.0f;
        for (int i = 0; i < 16; ++i) {
            const int level = clampi(nearest_int(inv_scale * v[i]), -32, 31);
            const float weight = v[i] * v[i];
            const float wv = weight * v[i];
            const float wvl = wv * (float)level;
            sum_lx = sum_lx + wvl;
            const float wll = weight * (float)(level * level);
            sum_l2 = sum_l2 + wll;
        }
        const float lhs = sum_lx * sum_lx;
        const float rhs = best * sum_l2;
        if (sum_l2 > 0.0f && lhs > rhs) {
            for (int i = 0; i < 16; ++i) levels[i] = clampi(nearest_int(inv_scale * v[i]), -32, 31) + 32;
            scale = sum_lx / sum_l2;
            best = scale * sum_lx;
        }
    }
    return scale;
}

// block = 64 threads = 4 superblocks, 16 lanes (one 16-value sub-block each) per superblock
__global__ __launch_bounds__(64) void quantize_q6_k_kernel(const float* __restrict__ x, uint8_t* __restrict__ out,
                                                           uint32_t k, uint64_t total_blocks) {
    __shared__ int lv[4][256];
    const int sbk = threadIdx.x >> 4;
    const uint64_t blk = (uint64_t)blockIdx.x * 4 + sbk;
    const int sub = threadIdx.x & 15;
    const int group_base = threadIdx.x & ~15;
    const bool active = blk < total_blocks;
    const uint32_t bpr = k / 256;
    float v[16];
    int levels[16];
    float bscale = 0.0f;
    if (active) {
        const uint64_t row = blk / bpr;
        const uint64_t b = blk % bpr;
        const float* src = x + row * k + b * 256 + sub * 16;
        for (int i = 0; i < 16; ++i) v[i] = src[i];
        bscale = make_qx_quants16(v, levels);
    }
    float max_scale = 0.0f, max_abs_scale = 0.0f;
    float scales[16];
    for (int j = 0; j < 16; ++j) {
        scales[j] = __shfl(bscale, group_base + j, 64);
        const float a = fabsf(scales[j]);
        if (a > max_abs_scale) {
            max_abs_scale = a;
            max_scale = scales[j];
        }
    }
    float d_scale;
    int code;
    if (max_abs_scale < 1.0e-12f) {
        d_scale = 0.0f;
        code = 0;
    } else {
        const float inv_scale = -128.0f / max_scale;
        d_scale = round_f16(1.0f / inv_scale);
        code = clampi(nearest_int(inv_scale * bscale), -128, 127);
    }
    if (active) {
        const float d = d_scale * (float)code;
        if (d != 0.0f) {
            for (int i = 0; i < 16; ++i) levels[i] = clampi(nearest_int(v[i] / d), -32, 31) + 32;
        }
        for (int i = 0; i < 16; ++i) lv[sbk][sub * 16 + i] = levels[i];
    }
    __syncthreads();
    if (!active) return;
    const int* L = lv[sbk];
    uint8_t* o = out + blk * 210;
    // 16 lanes write 210 bytes: ql 128, qh 64, scales 16, d 2
    for (int bidx = sub; bidx < 128; bidx += 16) {
        const int section = bidx >> 6;
        const int local = bidx & 31;
        const int base = section * 128;
        uint32_t byte;
        if ((bidx & 32) == 0) {
            byte = ((uint32_t)L[base + local] & 15u) | (((uint32_t)L[base + local + 64] & 15u) << 4);
        } else {
            byte = ((uint32_t)L[base + local + 32] & 15u) | (((uint32_t)L[base + local + 96] & 15u) << 4);
        }
        o[bidx] = (uint8_t)byte;
    }
    for (int bidx = sub; bidx < 64; bidx += 16) {
        const int section = bidx >> 5;
        const int local = bidx & 31;
        const int base = section * 128;
        const uint32_t byte = ((((uint32_t)L[base + local] & 63u) >> 4) & 3u) |
                              (((((uint32_t)L[base + local + 32] & 63u) >> 4) & 3u) << 2) |
                              (((((uint32_t)L[base + local + 64] & 63u) >> 4) & 3u) << 4) |
                              (((((uint32_t)L[base + local + 96] & 63u) >> 4) & 3u) << 6);
        o[128 + bidx] = (uint8_t)byte;
    }
    o[192 + sub] = (uint8_t)(code & 255);
    if (sub == 0) {
        const uint32_t d16 = f32_to_f16_bits_rne(d_scale);
        o[208] = (uint8_t)(d16 & 0xffu);
        o[209] = (uint8_t)(d16 >> 8);
    }
}

// ----------------------------------------------------------- dequantizers --
// One thread per output value; used to stage weights for the prefill GEMM
// checks and by tests.  Value order matches the CPU decoders.

__global__ void dequant_q4_k_kernel(const uint8_t* __restrict__ w, float* __restrict__ out, uint32_t k,
                                    uint64_t total) {
    const uint64_t idx = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= total) return;
    const uint64_t row = idx / k;
    const uint32_t col = (uint32_t)(idx % k);
    const uint8_t* blk = w + (row * (k / 256) + col / 256) * 144;
    const int i = col & 255;
    const int sb = i >> 5;
    uint32_t sc, m;
    if (sb < 4) {
        sc = blk[4 + sb] & 63u;
        m = blk[8 + sb] & 63u;
    } else {
        sc = (blk[12 + sb - 4] & 15u) | ((uint32_t)(blk[4 + sb - 4] >> 6) << 4);
        m = ((uint32_t)blk[12 + sb - 4] >> 4) | ((uint32_t)(blk[8 + sb - 4] >> 6) << 4);
    }
    const int byte = ((i >> 6) * 32) + (i & 31);
    const uint32_t q = (i & 32) ? ((uint32_t)blk[16 + byte] >> 4) : (blk[16 + byte] & 15u);
    const float d = f16_bits_to_f32(blk[0] | ((uint32_t)blk[1] << 8));
    const float dmin = f16_bits_to_f32(blk[2] | ((uint32_t)blk[3] << 8));
    const float a = d * (float)sc;
    const float a2 = a * (float)q;
    const float c = dmin * (float)m;
    out[idx] = a2 - c;
}

__global__ void dequant_q8_0_kernel(const uint8_t* __restrict__ w, float* __restrict__ out, uint32_t k,
                                    uint64_t total) {
    const uint64_t idx = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= total) return;
    const uint64_t row = idx / k;
    const uint32_t col = (uint32_t)(idx % k);
    const uint8_t* blk = w + (row * (k / 32) + col / 32) * 34;
    const float d = f16_bits_to_f32(blk[0] | ((uint32_t)blk[1] << 8));
    out[idx] = d * (float)(int8_t)blk[2 + (col & 31)];
}

__global__ void dequant_q6_k_kernel(const uint8_t* __restrict__ w, float* __restrict__ out, uint32_t k,
                                    uint64_t total) {
    const uint64_t idx = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= total) return;
    const uint64_t row = idx / k;
    const uint32_t col = (uint32_t)(idx % k);
    const uint8_t* blk = w + (row * (k / 256) + col / 256) * 210;
    const int i = col & 255;
    const int half = i >> 7, l = i & 127, quarter = l >> 5, pos = l & 31;
    const uint8_t* ql = blk + 64 * half;
    const uint8_t* qh = blk + 128 + 32 * half;
    uint32_t lo;
    if (quarter == 0) lo = ql[pos] & 15u;
    else if (quarter == 1) lo = ql[pos + 32] & 15u;
    else if (quarter == 2) lo = (uint32_t)ql[pos] >> 4;
    else lo = (uint32_t)ql[pos + 32] >> 4;
    const uint32_t hi = ((uint32_t)qh[pos] >> (2 * quarter)) & 3u;
    const int q = (int)(lo | (hi << 4)) - 32;
    const float d = f16_bits_to_f32(blk[208] | ((uint32_t)blk[209] << 8));
    const float a = d * (float)(int8_t)blk[192 + (i >> 4)];
    out[idx] = a * (float)q;
}

}  // namespace t2h

using namespace t2h;

static int quant_check(const void* x, const void* out, uint32_t rows, uint32_t k, uint32_t block) {
    if (!x || !out) return T2H_ERR_NULL;
    if (rows == 0 || k == 0 || k % block != 0) return T2H_ERR_SHAPE;
    return T2H_OK;
}

extern "C" int t2h_quantize_q8_0(const float* x, uint32_t rows, uint32_t k, void* out, void* stream) {
    int st = quant_check(x, out, rows, k, 32);
    if (st) return st;
    const uint64_t total = (uint64_t)rows * (k / 32);
    const uint64_t grid = (total + 1) / 2;
    if (grid > 0x7fffffffull) return T2H_ERR_SHAPE;
    hipLaunchKernelGGL(quantize_q8_0_kernel, dim3((uint32_t)grid), dim3(64), 0, (hipStream_t)stream, x,
                       (uint8_t*)out, k, total);
    T2H_LAUNCH_CHECK();
    return T2H_OK;
}

extern "C" int t2h_quantize_q4_k(const float* x, uint32_t rows, uint32_t k, void* out, void* stream) {
    int st = quant_check(x, out, rows, k, 256);
    if (st) return st;
    const uint64_t total = (uint64_t)rows * (k / 256);
    const uint64_t grid = (total + 7) / 8;
    if (grid > 0x7fffffffull) return T2H_ERR_SHAPE;
    hipLaunchKernelGGL(quantize_q4_k_kernel, dim3((uint32_t)grid), dim3(64), 0, (hipStream_t)stream, x,
                       (uint8_t*)out, k, total);
    T2H_LAUNCH_CHECK();
    return T2H_OK;
}

extern "C" int t2h_quantize_q6_k(const float* x, uint32_t rows, uint32_t k, void* out, void* stream) {
    int st = quant_check(x, out, rows, k, 256);
    if (st) return st;
    const uint64_t total = (uint64_t)rows * (k / 256);
    const uint64_t grid = (total + 3) / 4;
    if (grid > 0x7fffffffull) return T2H_ERR_SHAPE;
    hipLaunchKernelGGL(quantize_q6_k_kernel, dim3((uint32_t)grid), dim3(64), 0, (hipStream_t)stream, x,
                       (uint8_t*)out, k, total);
    T2H_LAUNCH_CHECK();
    return T2H_OK;
}

extern "C" int t2h_dequantize(int wtype, const void* w, uint32_t rows, uint32_t k, float* out, void* stream) {
    if (!w || !out) return T2H_ERR_NULL;
    const uint32_t block = wtype == T2H_WTYPE_Q8_0 ? 32u : 256u;
    if (rows == 0 || k == 0 || k % block) return T2H_ERR_SHAPE;
    const uint64_t total = (uint64_t)rows * k;
    const uint64_t grid = (total + 255) / 256;
    if (grid > 0x7fffffffull) return T2H_ERR_SHAPE;
    hipStream_t s = (hipStream_t)stream;
    switch (wtype) {
        case T2H_WTYPE_Q4_K:
            hipLaunchKernelGGL(dequant_q4_k_kernel, dim3((uint32_t)grid), dim3(256), 0, s, (const uint8_t*)w, out, k,
                               total);
            break;
        case T2H_WTYPE_Q6_K:
            hipLaunchKernelGGL(dequant_q6_k_kernel, dim3((uint32_t)grid), dim3(256), 0, s, (const uint8_t*)w, out, k,
                               total);
            break;
        case T2H_WTYPE_Q8_0:
            hipLaunchKernelGGL(dequant_q8_0_kernel, dim3((uint32_t)grid), dim3(256), 0, s, (const uint8_t*)w, out, k,
                               total);
            break;
        default:
            return T2H_ERR_ARG;
    }
    T2H_LAUNCH_CHECK();
    return T2H_OK;
}
