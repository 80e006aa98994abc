/*
 * CPU restatement of torch2vk's GGUF block quantizers and decoders.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity oracle for the HIP
 * quantizers and dequantizing kernels in torch2vk_amd/csrc.  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it, and
 * only as the checker.  The product path never calls into it.
 *
 * The reference quantizers are GLSL compute shaders that need a Vulkan
 * device.  This file restates them in the same fp32 operation order:
 *   - Q8_0: /root/reference/src/torch2vk/quantize/vulkan.py:143-182
 *   - Q4_K: /root/reference/src/torch2vk/quantize/vulkan.py:241-417
 *   - Q6_K: /root/reference/src/torch2vk/quantize/vulkan.py:479-634
 * GLSL leaves three things open that this restatement pins:
 *   - packHalf2x16 rounding: IEEE round-to-nearest-even, subnormals kept;
 *   - a*b+c is never contracted into an fma (build with -ffp-contract=off);
 *   - GLSL round() ties go to even (rintf in the default rounding mode).
 * Division and sqrt are the correctly rounded IEEE operations.
 *
 * Byte layouts (GGUF):
 *   Q8_0  34 B / 32 values:  fp16 d | 32 x int8
 *   Q4_K 144 B / 256 values: fp16 d | fp16 dmin | 12 B 6-bit scale/min codes | 128 B nibbles
 *   Q6_K 210 B / 256 values: 128 B ql | 64 B qh | 16 x int8 scales | fp16 d
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

/* ---------------------------------------------------------------- fp16 -- */

uint16_t oracle_f32_to_f16(float value) {
    uint32_t bits;
    memcpy(&bits, &value, 4);
    const uint32_t sign = (bits >> 16) & 0x8000u;
    const uint32_t exp = (bits >> 23) & 0xffu;
    uint32_t mant = bits & 0x7fffffu;
    if (exp == 0xffu) {
        return (uint16_t)(sign | 0x7c00u | (mant ? 0x200u : 0u));
    }
    int e = (int)exp - 127 + 15;
    if (e >= 31) {
        return (uint16_t)(sign | 0x7c00u);
    }
    if (e <= 0) {
        /* subnormal half (or zero): shift the full 24-bit significand */
        if (e < -10) {
            return (uint16_t)sign;
        }
        mant |= 0x800000u;
        const uint32_t shift = (uint32_t)(14 - e);
        uint32_t half_mant = mant >> shift;
        const uint32_t rem = mant & ((1u << shift) - 1u);
        const uint32_t halfway = 1u << (shift - 1u);
        if (rem > halfway || (rem == halfway && (half_mant & 1u))) {
            half_mant += 1u;
        }
        return (uint16_t)(sign | half_mant);
    }
    uint32_t half = ((uint32_t)e << 10) | (mant >> 13);
    const uint32_t rem = mant & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (half & 1u))) {
        half += 1u; /* may carry into the exponent, which is the correct result */
    }
    return (uint16_t)(sign | half);
}

float oracle_f16_to_f32(uint16_t half) {
    const uint32_t sign = ((uint32_t)half & 0x8000u) << 16;
    const uint32_t exp = ((uint32_t)half >> 10) & 0x1fu;
    uint32_t mant = (uint32_t)half & 0x3ffu;
    uint32_t bits;
    if (exp == 0) {
        if (mant == 0) {
            bits = sign;
        } else {
            int e = -1;
            do {
                e++;
                mant <<= 1;
            } while ((mant & 0x400u) == 0);
            mant &= 0x3ffu;
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | (mant << 13);
        }
    } else if (exp == 0x1fu) {
        bits = sign | 0x7f800000u | (mant << 13);
    } else {
        bits = sign | ((exp + 127u - 15u) << 23) | (mant << 13);
    }
    float out;
    memcpy(&out, &bits, 4);
    return out;
}

static float round_f16(float value) { return oracle_f16_to_f32(oracle_f32_to_f16(value)); }

/* GLSL clamp(x, lo, hi) == min(max(x, lo), hi) */
static float clampf(float x, float lo, float hi) { return fminf(fmaxf(x, lo), hi); }

/* ---------------------------------------------------------------- Q8_0 -- */

/* vulkan.py:143-148 */
static float round_away(float value) {
    const float absolute = fabsf(value);
    const float floored = floorf(absolute);
    const float rounded = floored + floorf(2.0f * (absolute - floored));
    const float s = value > 0.0f ? 1.0f : (value < 0.0f ? -1.0f : 0.0f);
    return s * rounded;
}

/* vulkan.py:150-182: one 32-value block -> 34 bytes */
static void q8_0_block(const float* values, uint8_t* out) {
    float amax = 0.0f;
    for (int i = 0; i < 32; ++i) {
        amax = fmaxf(amax, fabsf(values[i]));
    }
    const float block_scale = amax / 127.0f;
    const float inv_scale = block_scale == 0.0f ? 0.0f : 1.0f / block_scale;
    const uint16_t d16 = oracle_f32_to_f16(block_scale);
    out[0] = (uint8_t)(d16 & 0xffu);
    out[1] = (uint8_t)(d16 >> 8);
    for (int i = 0; i < 32; ++i) {
        int quant = (int)round_away(values[i] * inv_scale);
        if (quant < -128) quant = -128;
        if (quant > 127) quant = 127;
        out[2 + i] = (uint8_t)(quant & 255);
    }
}

void oracle_quantize_q8_0(const float* x, int64_t rows, int64_t k, uint8_t* out) {
    const int64_t blocks = k / 32;
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        for (int64_t b = 0; b < blocks; ++b) {
            q8_0_block(x + r * k + b * 32, out + (r * blocks + b) * 34);
        }
    }
}

/* ---------------------------------------------------------------- Q4_K -- */

/* vulkan.py:241-243 */
static uint32_t rounded_code(float value, uint32_t max_code) {
    return (uint32_t)clampf(floorf(value + 0.5f), 0.0f, (float)max_code);
}

/* vulkan.py:245-261 */
static float weighted_quant_error(const float* v, float scale, float minimum, float inv_scale) {
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

/* vulkan.py:263-329 */
static float choose_subblock_scale(const float* v, float* min_offset) {
    float min_value = v[0];
    float max_value = v[0];
    float sum_x2 = 0.0f;
    for (int i = 0; i < 32; ++i) {
        min_value = fminf(min_value, v[i]);
        max_value = fmaxf(max_value, v[i]);
        const float t = v[i] * v[i];
        sum_x2 = sum_x2 + t;
    }
    if (min_value > 0.0f) {
        min_value = 0.0f;
    }
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
        float sum_l = 0.0f;
        float sum_l2 = 0.0f;
        float sum_xl = 0.0f;
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

/* vulkan.py:352-417: one 256-value superblock -> 144 bytes */
static void q4_k_block(const float* values, uint8_t* out) {
    float subblock_scales[8];
    float subblock_mins[8];
    uint32_t scale_codes[8];
    uint32_t min_codes[8];
    uint32_t quants[256];
    for (int j = 0; j < 8; ++j) {
        float min_offset = 0.0f;
        subblock_scales[j] = choose_subblock_scale(values + 32 * j, &min_offset);
        subblock_mins[j] = min_offset;
    }
    float max_scale = 0.0f;
    float max_min = 0.0f;
    for (int j = 0; j < 8; ++j) {
        max_scale = fmaxf(max_scale, subblock_scales[j]);
        max_min = fmaxf(max_min, subblock_mins[j]);
    }
    float d_scale = max_scale > 0.0f ? max_scale / 63.0f : 0.0f;
    float d_min = max_min > 0.0f ? max_min / 63.0f : 0.0f;
    const float inv_scale = max_scale > 0.0f ? 63.0f / max_scale : 0.0f;
    const float inv_min = max_min > 0.0f ? 63.0f / max_min : 0.0f;
    for (int j = 0; j < 8; ++j) {
        scale_codes[j] = rounded_code(subblock_scales[j] * inv_scale, 63u);
        min_codes[j] = rounded_code(subblock_mins[j] * inv_min, 63u);
    }
    d_scale = round_f16(d_scale);
    d_min = round_f16(d_min);
    for (int lane = 0; lane < 256; ++lane) {
        const int sb = lane >> 5;
        const float scale = d_scale * (float)scale_codes[sb];
        const float minimum = d_min * (float)min_codes[sb];
        uint32_t quant = 0u;
        if (scale > 0.0f) {
            quant = rounded_code((values[lane] + minimum) / scale, 15u);
        }
        quants[lane] = quant;
    }
    const uint16_t d16 = oracle_f32_to_f16(d_scale);
    const uint16_t m16 = oracle_f32_to_f16(d_min);
    out[0] = (uint8_t)(d16 & 0xffu);
    out[1] = (uint8_t)(d16 >> 8);
    out[2] = (uint8_t)(m16 & 0xffu);
    out[3] = (uint8_t)(m16 >> 8);
    /* metadata_byte, vulkan.py:331-342 */
    for (int i = 0; i < 4; ++i) {
        out[4 + i] = (uint8_t)((scale_codes[i] & 63u) | ((scale_codes[i + 4] & 48u) << 2));
        out[8 + i] = (uint8_t)((min_codes[i] & 63u) | ((min_codes[i + 4] & 48u) << 2));
        out[12 + i] = (uint8_t)((scale_codes[i + 4] & 15u) | ((min_codes[i + 4] & 15u) << 4));
    }
    /* q_byte, vulkan.py:344-350 */
    for (int b = 0; b < 128; ++b) {
        const int group = b >> 5;
        const int local = b & 31;
        const uint32_t low = quants[group * 64 + local] & 15u;
        const uint32_t high = quants[group * 64 + 32 + local] & 15u;
        out[16 + b] = (uint8_t)(low | (high << 4));
    }
}

void oracle_quantize_q4_k(const float* x, int64_t rows, int64_t k, uint8_t* out) {
    const int64_t blocks = k / 256;
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        for (int64_t b = 0; b < blocks; ++b) {
            q4_k_block(x + r * k + b * 256, out + (r * blocks + b) * 144);
        }
    }
}

/* ---------------------------------------------------------------- Q6_K -- */

static int nearest_int(float value) { return (int)rintf(value); }

static int clampi(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }

/* vulkan.py:483-540 */
static float make_qx_quants16(const float* v, int* levels) {
    float max_value = 0.0f;
    float max_abs = 0.0f;
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
    float sum_lx = 0.0f;
    float sum_l2 = 0.0f;
    for (int i = 0; i < 16; ++i) {
        int level = clampi(nearest_int(inv_scale * v[i]), -32, 31);
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
            for (int i = 0; i < 16; ++i) {
                levels[i] = clampi(nearest_int(inv_scale * v[i]), -32, 31) + 32;
            }
            scale = sum_lx / sum_l2;
            best = scale * sum_lx;
        }
    }
    return scale;
}

/* The per-sub-block searches on their own, over n sub-blocks (32 values for Q4_K, 16 for Q6_K), so that tests
 * can check which candidate each one keeps. */
void oracle_q4_k_subblocks(const float* v, int64_t n, float* scales, float* min_offsets) {
    for (int64_t i = 0; i < n; ++i) scales[i] = choose_subblock_scale(v + 32 * i, min_offsets + i);
}

void oracle_q6_k_subblocks(const float* v, int64_t n, float* scales, int* levels) {
    for (int64_t i = 0; i < n; ++i) scales[i] = make_qx_quants16(v + 16 * i, levels + 16 * i);
}

/* vulkan.py:566-634: one 256-value superblock -> 210 bytes */
static void q6_k_block(const float* values, uint8_t* out) {
    int levels[256];
    float block_scales[16];
    int scale_codes[16];
    for (int j = 0; j < 16; ++j) {
        block_scales[j] = make_qx_quants16(values + 16 * j, levels + 16 * j);
    }
    float max_scale = 0.0f;
    float max_abs_scale = 0.0f;
    for (int j = 0; j < 16; ++j) {
        const float a = fabsf(block_scales[j]);
        if (a > max_abs_scale) {
            max_abs_scale = a;
            max_scale = block_scales[j];
        }
    }
    float d_scale;
    if (max_abs_scale < 1.0e-12f) {
        d_scale = 0.0f;
        for (int j = 0; j < 16; ++j) scale_codes[j] = 0;
    } else {
        const float inv_scale = -128.0f / max_scale;
        d_scale = round_f16(1.0f / inv_scale);
        for (int j = 0; j < 16; ++j) {
            scale_codes[j] = clampi(nearest_int(inv_scale * block_scales[j]), -128, 127);
        }
    }
    for (int j = 0; j < 16; ++j) {
        const float d = d_scale * (float)scale_codes[j];
        if (d != 0.0f) {
            for (int i = 0; i < 16; ++i) {
                levels[16 * j + i] = clampi(nearest_int(values[16 * j + i] / d), -32, 31) + 32;
            }
        }
    }
    /* ql_byte, vulkan.py:546-554 */
    for (int b = 0; b < 128; ++b) {
        const int section = b >> 6;
        const int local = b & 31;
        const int base = section * 128;
        uint32_t byte;
        if ((b & 32) == 0) {
            byte = ((uint32_t)levels[base + local] & 15u) | (((uint32_t)levels[base + local + 64] & 15u) << 4);
        } else {
            byte = ((uint32_t)levels[base + local + 32] & 15u) | (((uint32_t)levels[base + local + 96] & 15u) << 4);
        }
        out[b] = (uint8_t)byte;
    }
    /* qh_byte, vulkan.py:556-564 */
    for (int b = 0; b < 64; ++b) {
        const int section = b >> 5;
        const int local = b & 31;
        const int base = section * 128;
        const uint32_t byte = ((((uint32_t)levels[base + local] & 63u) >> 4) & 3u) |
                              (((((uint32_t)levels[base + local + 32] & 63u) >> 4) & 3u) << 2) |
                              (((((uint32_t)levels[base + local + 64] & 63u) >> 4) & 3u) << 4) |
                              (((((uint32_t)levels[base + local + 96] & 63u) >> 4) & 3u) << 6);
        out[128 + b] = (uint8_t)byte;
    }
    for (int j = 0; j < 16; ++j) {
        out[192 + j] = (uint8_t)(scale_codes[j] & 255);
    }
    const uint16_t d16 = oracle_f32_to_f16(d_scale);
    out[208] = (uint8_t)(d16 & 0xffu);
    out[209] = (uint8_t)(d16 >> 8);
}

void oracle_quantize_q6_k(const float* x, int64_t rows, int64_t k, uint8_t* out) {
    const int64_t blocks = k / 256;
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        for (int64_t b = 0; b < blocks; ++b) {
            q6_k_block(x + r * k + b * 256, out + (r * blocks + b) * 210);
        }
    }
}

/* ------------------------------------------------------------ decoders -- */

/* Q4_K value, following the embedding decoder's fp32 order:
 * dm.x * float(scale) * float(q) - dm.y * float(minimum)
 * (/root/reference/src/models/quantized_qwen3/shaders/embedding_q4_k_f32.py:97-110) */
void oracle_dequant_q4_k(const uint8_t* w, int64_t rows, int64_t k, float* out) {
    const int64_t blocks = k / 256;
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        for (int64_t b = 0; b < blocks; ++b) {
            const uint8_t* blk = w + (r * blocks + b) * 144;
            const float d = oracle_f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
            const float dmin = oracle_f16_to_f32((uint16_t)(blk[2] | (blk[3] << 8)));
            for (int i = 0; i < 256; ++i) {
                const int sb = i >> 5;
                uint32_t sc, m;
                if (sb < 4) {
                    sc = blk[4 + sb] & 63u;
                    m = blk[8 + sb] & 63u;
                } else {
                    sc = (blk[12 + sb - 4] & 15u) | ((blk[4 + sb - 4] >> 6) << 4);
                    m = (blk[12 + sb - 4] >> 4) | ((blk[8 + sb - 4] >> 6) << 4);
                }
                const int byte = ((i >> 6) * 32) + (i & 31);
                const uint32_t q = (i & 32) ? (blk[16 + byte] >> 4) : (blk[16 + byte] & 15u);
                const float a = d * (float)sc;
                const float a2 = a * (float)q;
                const float c = dmin * (float)m;
                out[r * k + b * 256 + i] = a2 - c;
            }
        }
    }
}

/* Q6_K value: d * float(scale_j) * float(q - 32)
 * (decoder: /root/reference/src/models/quantized_qwen3/shaders/linear_nobias_q6_k_matvec_f32.py:116-156) */
void oracle_dequant_q6_k(const uint8_t* w, int64_t rows, int64_t k, float* out) {
    const int64_t blocks = k / 256;
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        for (int64_t b = 0; b < blocks; ++b) {
            const uint8_t* blk = w + (r * blocks + b) * 210;
            const float d = oracle_f16_to_f32((uint16_t)(blk[208] | (blk[209] << 8)));
            for (int i = 0; i < 256; ++i) {
                const int half = i >> 7;      /* 128-value half */
                const int l = i & 127;
                const int quarter = l >> 5;   /* 0..3 */
                const int pos = l & 31;
                const uint8_t* ql = blk + 64 * half;
                const uint8_t* qh = blk + 128 + 32 * half;
                uint32_t lo;
                if (quarter == 0) lo = ql[pos] & 15u;
                else if (quarter == 1) lo = ql[pos + 32] & 15u;
                else if (quarter == 2) lo = ql[pos] >> 4;
                else lo = ql[pos + 32] >> 4;
                const uint32_t hi = (qh[pos] >> (2 * quarter)) & 3u;
                const int q = (int)(lo | (hi << 4)) - 32;
                const int8_t sc = (int8_t)blk[192 + (i >> 4)];
                const float a = d * (float)sc;
                out[r * k + b * 256 + i] = a * (float)q;
            }
        }
    }
}

/* Q8_0 value: d * float(int8)
 * (/root/reference/src/models/quantized_qwen3/shaders/linear_nobias_q8_0_matvec_f32.py:84-95) */
void oracle_dequant_q8_0(const uint8_t* w, int64_t rows, int64_t k, float* out) {
    const int64_t blocks = k / 32;
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        for (int64_t b = 0; b < blocks; ++b) {
            const uint8_t* blk = w + (r * blocks + b) * 34;
            const float d = oracle_f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
            for (int i = 0; i < 32; ++i) {
                out[r * k + b * 32 + i] = d * (float)(int8_t)blk[2 + i];
            }
        }
    }
}
