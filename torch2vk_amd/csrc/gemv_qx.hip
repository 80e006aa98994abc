// Q6_K and Q8_0 dequant-GEMV for decode (M = 1 token), gfx950.
//
// Replaces the reference's matvec shaders for the two other GGUF types the
// Q4_K_M policy and the K % 256 != 0 rule select:
//   LINEAR_NOBIAS_Q6_K_MATVEC_F32     (src/models/quantized_qwen3/shaders/linear_nobias_q6_k_matvec_f32.py:20-193)
//   LINEAR_NOBIAS_Q6_K_MATVEC_ADD_F32 (src/models/optimized_qwen3/shaders/linear_nobias_q6_k_matvec_add_f32.py:23-100)
//   LINEAR_NOBIAS_Q8_0_MATVEC_F32     (src/models/quantized_qwen3/shaders/linear_nobias_q8_0_matvec_f32.py:24-119)
//   LM_HEAD_Q6_K_ARGMAX_PARTIAL_F16   (src/torch2vk/export/shaders/lm_head_q6_k_argmax_partial_f16.py:24-209)
//   + RMS_NORM_MUL_F16_F32 fused as a prologue (v_proj of the more-bits layers, the LM head).
//
// Block formats (GGUF):
//   Q6_K, 210 B / 256 values: ql[128] low nibbles | qh[64] high 2-bit pairs |
//         int8 scales[16] (one per 16 values) | fp16 d;
//         value(128h + 32p + l) = d * sc[8h + 2p + l/16] * (q - 32),
//         q = (ql[64h + 32(p&1) + l] >> 4(p>>1) & 15) | ((qh[32h + l] >> 2p) & 3) << 4
//   Q8_0, 34 B / 32 values: fp16 d | int8 q[32]; value = d * q.
// Rows are NB * block bytes long, so blocks are only halfword aligned; the
// 16-B loads below rely on the hardware's unaligned access.
//
// Work mapping.  A row is cut into "pieces": a quarter of a Q6_K superblock
// (64 values: 16 of each of its 4 parts) or one Q8_0 block (32 values).  A
// wave covers a unit of RPW rows with NIT steps of 64 pieces, lane l taking
// flat piece it*64 + l, so each lane always meets the same columns.  x is
// staged once per 512-thread block in LDS as pair words (e0,e2),(e1,e3) that
// line up with the and-or weight expansion below, plus fp32 sums of every 16
// values.  A lane's x slices do not change from unit to unit, so the compiler
// keeps them in registers after one read from LDS.
//
// Arithmetic.  6-bit Q6_K codes q become bf16 128+q (0x4300 | q) and 8-bit
// Q8_0 codes become fp16 1024+(q+128) (0x6400 | (q ^ 0x80)), so one and-or
// builds two operands of v_dot2; the offsets come off with the x sums:
//   Q6_K: sum x*(q-32)  = sum x*(128+q) - 160 * sum x
//   Q8_0: sum x*q       = sum x*(1024+q+128) - 1152 * sum x
// Q8_0 runs on fp16 x (the reference's activation type); every product is
// exact in fp32 and the offset cancels to within a few fp32 ulps of the sum.
#include "common.h"

namespace t2h {

enum QxPrologue { QXPRO_BF16 = 0, QXPRO_RMSNORM = 1 };
enum QxEpilogue { QXEPI_F32 = 0, QXEPI_BF16 = 1, QXEPI_RESID = 2, QXEPI_ARGMAX = 4 };

struct QxArgs {
    const void* x;          // QXPRO_BF16: bf16 [K];  QXPRO_RMSNORM: fp32 [K]
    const float* norm_w;    // QXPRO_RMSNORM: fp32 [K]
    const float* residual;  // QXEPI_RESID: fp32 [N] (may alias y)
    const uint8_t* w;
    void* y;
    uint32_t k;
    uint32_t row_bytes;
    uint32_t pieces;          // pieces per row
    uint32_t n_units;         // units of RPW rows
    uint32_t units_per_wave;
    float* partial_scores;    // QXEPI_ARGMAX: [gridDim.x]
    uint32_t* partial_tokens;
    float eps;
};

constexpr int QX_THREADS = 512;
constexpr uint32_t QX_WAVES = QX_THREADS / 64;

// ---------------------------------------------------------------- Q6_K ----

struct Q6KFormat {
    static constexpr int BLOCK_VALUES = 256;
    static constexpr int BLOCK_BYTES = 210;
    static constexpr int PIECES = 4;  // pieces per block
    static constexpr bool X_F16 = false;
    static constexpr uint32_t MAX_NIT = 3;  // x slices stay in registers: 36 VGPRs per step
    struct Raw {
        uint4 ql0, ql1, qh;
        uint2 sc;
        uint32_t d;
    };
    // piece sub = 2h + (l0/16): half h of the superblock, values l0..l0+15 of each part
    __device__ static __forceinline__ void load(const uint8_t* blk, int sub, Raw& r) {
        const int h = sub >> 1;
        const int l0 = (sub & 1) * 16;
        r.d = load_u16(blk + 208);
        r.sc = load_u2_ua(blk + 192 + 8 * h);
        r.qh = load_u4_ua(blk + 128 + 32 * h + l0);
        r.ql0 = load_u4_ua(blk + 64 * h + l0);
        r.ql1 = load_u4_ua(blk + 64 * h + 32 + l0);
    }
    // first value of part 0 of this piece within the row
    __device__ static __forceinline__ int first_value(int blk, int sub) {
        return blk * 256 + 128 * (sub >> 1) + 16 * (sub & 1);
    }
    __device__ static __forceinline__ float dot(const Raw& r, const uint32_t* xw, const float* xs, int e0, int sub) {
        const uint32_t ql0[4] = {r.ql0.x, r.ql0.y, r.ql0.z, r.ql0.w};
        const uint32_t ql1[4] = {r.ql1.x, r.ql1.y, r.ql1.z, r.ql1.w};
        const uint32_t qh[4] = {r.qh.x, r.qh.y, r.qh.z, r.qh.w};
        const uint32_t B = 0x43004300u, LO = 0x000f000fu, HI = 0x00300030u;
        const uint32_t* x0 = xw + (e0 >> 1);  // part p pairs start 16 words later per part
        float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f, s3 = 0.0f;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const uint32_t w0 = ql0[c], w1 = ql1[c], hq = qh[c];
            s0 = dot2_bf16((w0 & LO) | ((hq << 4) & HI) | B, x0[2 * c], s0);
            s0 = dot2_bf16(((w0 >> 8) & LO) | ((hq >> 4) & HI) | B, x0[2 * c + 1], s0);
            s1 = dot2_bf16((w1 & LO) | ((hq << 2) & HI) | B, x0[16 + 2 * c], s1);
            s1 = dot2_bf16(((w1 >> 8) & LO) | ((hq >> 6) & HI) | B, x0[16 + 2 * c + 1], s1);
            s2 = dot2_bf16(((w0 >> 4) & LO) | (hq & HI) | B, x0[32 + 2 * c], s2);
            s2 = dot2_bf16(((w0 >> 12) & LO) | ((hq >> 8) & HI) | B, x0[32 + 2 * c + 1], s2);
            s3 = dot2_bf16(((w1 >> 4) & LO) | ((hq >> 2) & HI) | B, x0[48 + 2 * c], s3);
            s3 = dot2_bf16(((w1 >> 12) & LO) | ((hq >> 10) & HI) | B, x0[48 + 2 * c + 1], s3);
        }
        const float* xsum = xs + (e0 >> 4);  // 16-value sums; parts are 2 sums apart
        // int8 scales sc[8h + 2p + (sub & 1)]: bytes (sub&1) and 2+(sub&1) of each dword
        const int sh = (sub & 1) * 8;
        const uint32_t c0 = r.sc.x >> sh, c1 = r.sc.y >> sh;
        const float sc0 = (float)(int8_t)(c0 & 0xffu);
        const float sc1 = (float)(int8_t)((c0 >> 16) & 0xffu);
        const float sc2 = (float)(int8_t)(c1 & 0xffu);
        const float sc3 = (float)(int8_t)((c1 >> 16) & 0xffu);
        float t = sc0 * fmaf(-160.0f, xsum[0], s0);
        t = fmaf(sc1, fmaf(-160.0f, xsum[2], s1), t);
        t = fmaf(sc2, fmaf(-160.0f, xsum[4], s2), t);
        t = fmaf(sc3, fmaf(-160.0f, xsum[6], s3), t);
        return f16_bits_to_f32(r.d) * t;
    }
};

// ---------------------------------------------------------------- Q8_0 ----

struct Q80Format {
    static constexpr int BLOCK_VALUES = 32;
    static constexpr int BLOCK_BYTES = 34;
    static constexpr int PIECES = 1;
    static constexpr bool X_F16 = true;
    static constexpr uint32_t MAX_NIT = 6;  // 17 VGPRs of x per step
    struct Raw {
        uint4 q0, q1;
        uint32_t d;
    };
    __device__ static __forceinline__ void load(const uint8_t* blk, int, Raw& r) {
        r.d = load_u16(blk);
        r.q0 = load_u4_ua(blk + 2);
        r.q1 = load_u4_ua(blk + 18);
    }
    __device__ static __forceinline__ int first_value(int blk, int) { return blk * 32; }
    __device__ static __forceinline__ float dot(const Raw& r, const uint32_t* xw, const float* xs, int e0, int) {
        const uint32_t q[8] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w, r.q1.x, r.q1.y, r.q1.z, r.q1.w};
        const uint32_t B = 0x64006400u, M = 0x00ff00ffu;
        const uint32_t* x0 = xw + (e0 >> 1);
        float sa = 0.0f, sb = 0.0f;
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            const uint32_t w = q[c] ^ 0x80808080u;  // int8 q -> q + 128 in [0, 255]
            sa = dot2_f16((w & M) | B, x0[2 * c], sa);
            sb = dot2_f16(((w >> 8) & M) | B, x0[2 * c + 1], sb);
        }
        const float xsum = xs[e0 >> 4] + xs[(e0 >> 4) + 1];
        return f16_bits_to_f32(r.d) * fmaf(-1152.0f, xsum, sa + sb);
    }
};

// ----------------------------------------------------------- x staging ----

// 8 consecutive values -> 4 pair words (e0,e2),(e1,e3),(e4,e6),(e5,e7) of
// 16-bit codes (bf16 or fp16) plus the fp32 sum of the rounded values.
template <bool F16>
__device__ __forceinline__ void stage8(const float (&v)[8], uint32_t* dst, float& sum) {
    uint32_t c[8];
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        if constexpr (F16) {
            c[i] = f32_to_f16_bits_rne(v[i]);
            s += f16_bits_to_f32(c[i]);
        } else {
            c[i] = f32_to_bf16_bits(v[i]);
            s += bf16_bits_to_f32(c[i]);
        }
    }
    *reinterpret_cast<uint4*>(dst) =
        make_uint4(c[0] | (c[2] << 16), c[1] | (c[3] << 16), c[4] | (c[6] << 16), c[5] | (c[7] << 16));
    sum = s;
}

template <class F, int PRO, int EPI, int RPW, int NIT>
__global__ __launch_bounds__(QX_THREADS) void qx_gemv_kernel(const QxArgs a) {
    extern __shared__ __align__(16) uint32_t qx_lds[];
    const int K = (int)a.k;
    uint32_t* xw = qx_lds;                                   // K/2 pair words
    float* xs = reinterpret_cast<float*>(qx_lds + K / 2);    // K/16 sums

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int tid = threadIdx.x;

    // ------------------------------------------------------------ x stage --
    float inv = 1.0f;
    if constexpr (PRO == QXPRO_RMSNORM) {
        __shared__ float red[QX_WAVES];
        const float* h = reinterpret_cast<const float*>(a.x);
        float ss = 0.0f;
        for (int k = tid * 4; k < K; k += QX_THREADS * 4) {
            const float4 v = *reinterpret_cast<const float4*>(h + k);
            ss = fmaf(v.x, v.x, ss);
            ss = fmaf(v.y, v.y, ss);
            ss = fmaf(v.z, v.z, ss);
            ss = fmaf(v.w, v.w, ss);
        }
        ss = wave_sum(ss);
        if (lane == 0) red[wave] = ss;
        __syncthreads();
        float total = 0.0f;
#pragma unroll
        for (int i = 0; i < (int)QX_WAVES; ++i) total += red[i];
        inv = 1.0f / sqrtf(total / (float)K + a.eps);
    }
    // K % 16 == 0, so chunks c and c^1 (one 16-value sum) are always both live
    for (int c = tid; c < K / 8; c += QX_THREADS) {
        float v[8];
        if constexpr (PRO == QXPRO_RMSNORM) {
            const float* h = reinterpret_cast<const float*>(a.x) + c * 8;
            const float* nw = a.norm_w + c * 8;
            const float4 h0 = *reinterpret_cast<const float4*>(h), h1 = *reinterpret_cast<const float4*>(h + 4);
            const float4 w0 = *reinterpret_cast<const float4*>(nw), w1 = *reinterpret_cast<const float4*>(nw + 4);
            v[0] = h0.x * inv * w0.x; v[1] = h0.y * inv * w0.y; v[2] = h0.z * inv * w0.z; v[3] = h0.w * inv * w0.w;
            v[4] = h1.x * inv * w1.x; v[5] = h1.y * inv * w1.y; v[6] = h1.z * inv * w1.z; v[7] = h1.w * inv * w1.w;
        } else {
            const uint4 r = load_u4(reinterpret_cast<const uint16_t*>(a.x) + c * 8);
            const uint32_t u[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                v[2 * i] = bf16_bits_to_f32(u[i] & 0xffffu);
                v[2 * i + 1] = bf16_bits_to_f32(u[i] >> 16);
            }
        }
        float s;
        stage8<F::X_F16>(v, xw + c * 4, s);
        s += __shfl_xor(s, 1, T2H_WAVE);
        if ((c & 1) == 0) xs[c >> 1] = s;
    }
    __syncthreads();

    // --------------------------------------------------------- pieces -----
    const uint32_t P = a.pieces;
    int rloc[NIT], sub[NIT], e0[NIT];
    uint32_t woff[NIT];
    bool on[NIT];
#pragma unroll
    for (int it = 0; it < NIT; ++it) {
        const uint32_t f = (uint32_t)(it * 64 + lane);
        on[it] = f < RPW * P;
        const uint32_t ff = on[it] ? f : 0u;
        const uint32_t r = ff / P, p = ff % P;
        const int blk = (int)(p / F::PIECES);
        rloc[it] = (int)r;
        sub[it] = (int)(p % F::PIECES);
        e0[it] = F::first_value(blk, sub[it]);
        woff[it] = r * a.row_bytes + (uint32_t)blk * F::BLOCK_BYTES;
    }

    constexpr int NSTAGE = NIT <= 3 ? 2 : 1;
    typename F::Raw st[NSTAGE][NIT];
    const uint32_t wave_global = blockIdx.x * QX_WAVES + wave;
    const uint32_t total_waves = gridDim.x * QX_WAVES;
    const uint32_t last_unit = a.n_units - 1;
    auto clamp_unit = [&](uint32_t u) { return u < a.n_units ? u : last_unit; };
    auto issue = [&](uint32_t unit, typename F::Raw (&raw)[NIT]) {
        const uint8_t* base = a.w + (size_t)unit * RPW * a.row_bytes;
#pragma unroll
        for (int it = 0; it < NIT; ++it) F::load(base + woff[it], sub[it], raw[it]);
    };

    float best_score = -3.4028234663852886e38f;
    uint32_t best_token = 0xffffffffu;
    auto consume = [&](uint32_t u, const typename F::Raw (&raw)[NIT]) {
        float acc[RPW];
#pragma unroll
        for (int r = 0; r < RPW; ++r) acc[r] = 0.0f;
#pragma unroll
        for (int it = 0; it < NIT; ++it) {
            float c = F::dot(raw[it], xw, xs, e0[it], sub[it]);
            c = on[it] ? c : 0.0f;
            if constexpr (RPW == 1) {
                acc[0] += c;
            } else {
#pragma unroll
                for (int r = 0; r < RPW; ++r) acc[r] += (rloc[it] == r) ? c : 0.0f;
            }
        }
        float res[RPW];
#pragma unroll
        for (int r = 0; r < RPW; ++r) res[r] = wave_sum(acc[r]);
        if (u >= a.n_units) return;
        const uint32_t row0 = u * RPW;
        if constexpr (EPI == QXEPI_ARGMAX) {
#pragma unroll
            for (int r = 0; r < RPW; ++r) {
                if (better_pair(res[r], row0 + r, best_score, best_token)) {
                    best_score = res[r];
                    best_token = row0 + r;
                }
            }
        } else if (lane < RPW) {
            float v = res[0];
#pragma unroll
            for (int r = 1; r < RPW; ++r) v = (lane == r) ? res[r] : v;
            const uint32_t row = row0 + lane;
            if constexpr (EPI == QXEPI_F32) {
                reinterpret_cast<float*>(a.y)[row] = v;
            } else if constexpr (EPI == QXEPI_BF16) {
                reinterpret_cast<uint16_t*>(a.y)[row] = (uint16_t)f32_to_bf16_bits(v);
            } else if constexpr (EPI == QXEPI_RESID) {
                reinterpret_cast<float*>(a.y)[row] = a.residual[row] + v;
            }
        }
    };

    const uint32_t n_iter = (a.units_per_wave + NSTAGE - 1) / NSTAGE * NSTAGE;
    if constexpr (NSTAGE == 1) {
        for (uint32_t i = 0; i < n_iter; ++i) {
            issue(clamp_unit(wave_global + i * total_waves), st[0]);
            consume(wave_global + i * total_waves, st[0]);
        }
    } else {
        issue(clamp_unit(wave_global), st[0]);
        for (uint32_t i = 0; i < n_iter; i += 2) {
            issue(clamp_unit(wave_global + (i + 1) * total_waves), st[1]);
            consume(wave_global + i * total_waves, st[0]);
            if (i + 2 < n_iter) issue(clamp_unit(wave_global + (i + 2) * total_waves), st[0]);
            consume(wave_global + (i + 1) * total_waves, st[1]);
        }
    }

    if constexpr (EPI == QXEPI_ARGMAX) {
        __shared__ float bs[QX_WAVES];
        __shared__ uint32_t bt[QX_WAVES];
        if (lane == 0) {
            bs[wave] = best_score;
            bt[wave] = best_token;
        }
        __syncthreads();
        if (tid == 0) {
            float s = bs[0];
            uint32_t t = bt[0];
            for (int i = 1; i < (int)QX_WAVES; ++i) {
                if (better_pair(bs[i], bt[i], s, t)) {
                    s = bs[i];
                    t = bt[i];
                }
            }
            a.partial_scores[blockIdx.x] = s;
            a.partial_tokens[blockIdx.x] = t;
        }
    }
}

// ----------------------------------------------------------------- host ---

struct QxGeom {
    uint32_t pieces, rpw, nit;
};

// RPW rows per unit so that short rows still fill the 64 lanes, NIT steps of
// 64 pieces per unit (rounded up to an instantiated count).
template <class F>
static int qx_geometry(uint32_t k, QxGeom& g) {
    if (k == 0 || k % F::BLOCK_VALUES != 0 || k % 16 != 0) return T2H_ERR_SHAPE;
    const uint32_t piece_values = F::BLOCK_VALUES / F::PIECES;
    g.pieces = k / piece_values;
    g.rpw = (g.pieces < 64 && 64 % g.pieces == 0) ? 64 / g.pieces : 1;
    if (g.rpw > 4) return T2H_ERR_UNSUPPORTED;
    const uint32_t nit = (g.rpw * g.pieces + 63) / 64;
    static const uint32_t built[] = {1, 2, 3, 4, 6, 8};
    g.nit = 0;
    for (uint32_t b : built) {
        if (nit <= b) {
            g.nit = b;
            break;
        }
    }
    if (g.nit == 0 || g.nit > F::MAX_NIT) return T2H_ERR_UNSUPPORTED;
    if ((size_t)k * 2 + (size_t)k / 16 * 4 > 64 * 1024) return T2H_ERR_UNSUPPORTED;
    return T2H_OK;
}

template <class F, int PRO, int EPI>
static hipError_t qx_launch_geom(const QxGeom& g, dim3 grid, const QxArgs& a, hipStream_t s) {
    const size_t lds = (size_t)a.k * 2 + (size_t)a.k / 16 * 4;
    const dim3 block(QX_THREADS);
#define T2H_QX_CASE(R, I)                                                                      \
    if constexpr (I <= F::MAX_NIT) {                                                           \
        if (g.rpw == R && g.nit == I) {                                                        \
            hipLaunchKernelGGL((qx_gemv_kernel<F, PRO, EPI, R, I>), grid, block, lds, s, a);   \
            return hipGetLastError();                                                          \
        }                                                                                      \
    }
    T2H_QX_CASE(4, 1)
    T2H_QX_CASE(2, 1)
    T2H_QX_CASE(1, 1)
    T2H_QX_CASE(1, 2)
    T2H_QX_CASE(1, 3)
    T2H_QX_CASE(1, 4)
    T2H_QX_CASE(1, 6)
    T2H_QX_CASE(1, 8)
#undef T2H_QX_CASE
    return hipErrorInvalidValue;
}

static uint32_t qx_units_per_wave(uint32_t n_units, uint32_t blocks) {
    const uint32_t waves = blocks * QX_WAVES;
    return (n_units + waves - 1u) / waves;
}

static uint32_t qx_pick_blocks(uint32_t n_units, uint32_t max_blocks) {
    const uint32_t u = qx_units_per_wave(n_units, max_blocks);
    uint32_t blocks = (n_units + QX_WAVES * u - 1u) / (QX_WAVES * u);
    return blocks ? blocks : 1u;
}

constexpr uint32_t QX_MAX_BLOCKS = 256;

template <class F>
static int qx_run(int pro, int epi, QxArgs a, const QxGeom& g, uint32_t n, uint32_t blocks, hipStream_t s) {
    if (n % g.rpw != 0) return T2H_ERR_SHAPE;
    a.pieces = g.pieces;
    a.row_bytes = a.k / F::BLOCK_VALUES * F::BLOCK_BYTES;
    a.n_units = n / g.rpw;
    if (a.n_units == 0) return T2H_OK;
    if (blocks == 0) blocks = qx_pick_blocks(a.n_units, QX_MAX_BLOCKS);
    a.units_per_wave = qx_units_per_wave(a.n_units, blocks);
    const dim3 grid(blocks);
    hipError_t e = hipErrorInvalidValue;
    if (pro == QXPRO_BF16) {
        switch (epi) {
            case QXEPI_F32: e = qx_launch_geom<F, QXPRO_BF16, QXEPI_F32>(g, grid, a, s); break;
            case QXEPI_BF16: e = qx_launch_geom<F, QXPRO_BF16, QXEPI_BF16>(g, grid, a, s); break;
            case QXEPI_RESID: e = qx_launch_geom<F, QXPRO_BF16, QXEPI_RESID>(g, grid, a, s); break;
            case QXEPI_ARGMAX: e = qx_launch_geom<F, QXPRO_BF16, QXEPI_ARGMAX>(g, grid, a, s); break;
            default: return T2H_ERR_ARG;
        }
    } else {
        switch (epi) {
            case QXEPI_F32: e = qx_launch_geom<F, QXPRO_RMSNORM, QXEPI_F32>(g, grid, a, s); break;
            case QXEPI_BF16: e = qx_launch_geom<F, QXPRO_RMSNORM, QXEPI_BF16>(g, grid, a, s); break;
            case QXEPI_ARGMAX: e = qx_launch_geom<F, QXPRO_RMSNORM, QXEPI_ARGMAX>(g, grid, a, s); break;
            default: return T2H_ERR_ARG;
        }
    }
    return e == hipSuccess ? T2H_OK : T2H_ERR_HIP_BASE + (int)e;
}

// y = [RMSNorm](x) . deq(W)^T [+ residual], one launch per token row
template <class F>
static int qx_matvec(const void* x, const float* norm_w, float eps, const void* w, void* y, int out_dtype,
                     const float* residual, uint32_t m, uint32_t k, uint32_t n, void* stream) {
    if (!x || !w || !y) return T2H_ERR_NULL;
    QxGeom g;
    int st = qx_geometry<F>(k, g);
    if (st) return st;
    if (m == 0 || n == 0) return T2H_OK;
    if (n % g.rpw != 0) return T2H_ERR_SHAPE;
    int epi;
    if (residual) {
        if (out_dtype != T2H_DTYPE_F32 || norm_w) return T2H_ERR_DTYPE;
        epi = QXEPI_RESID;
    } else if (out_dtype == T2H_DTYPE_F32) {
        epi = QXEPI_F32;
    } else if (out_dtype == T2H_DTYPE_BF16) {
        epi = QXEPI_BF16;
    } else {
        return T2H_ERR_DTYPE;
    }
    const size_t x_size = norm_w ? 4 : 2;
    const size_t out_size = out_dtype == T2H_DTYPE_F32 ? 4 : 2;
    for (uint32_t row = 0; row < m; ++row) {
        QxArgs a = {};
        a.x = reinterpret_cast<const uint8_t*>(x) + (size_t)row * k * x_size;
        a.norm_w = norm_w;
        a.eps = eps;
        a.residual = residual ? residual + (size_t)row * n : nullptr;
        a.w = reinterpret_cast<const uint8_t*>(w);
        a.y = reinterpret_cast<uint8_t*>(y) + (size_t)row * n * out_size;
        a.k = k;
        st = qx_run<F>(norm_w ? QXPRO_RMSNORM : QXPRO_BF16, epi, a, g, n, 0, reinterpret_cast<hipStream_t>(stream));
        if (st) return st;
    }
    return T2H_OK;
}

}  // namespace t2h

using namespace t2h;

namespace t2h {
bool q4k_matvec_shape_built(uint32_t k, uint32_t n);
}

extern "C" int t2h_matvec_supported(int wtype, uint32_t k, uint32_t n) {
    QxGeom g;
    switch (wtype) {
        case T2H_WTYPE_Q4_K: return q4k_matvec_shape_built(k, n) ? 1 : 0;
        case T2H_WTYPE_Q6_K: return n > 0 && qx_geometry<Q6KFormat>(k, g) == T2H_OK && n % g.rpw == 0 ? 1 : 0;
        case T2H_WTYPE_Q8_0: return n > 0 && qx_geometry<Q80Format>(k, g) == T2H_OK && n % g.rpw == 0 ? 1 : 0;
        default: return 0;
    }
}

extern "C" int t2h_q6k_matvec(const void* x, const void* w, void* y, int out_dtype, const float* residual,
                              uint32_t m, uint32_t k, uint32_t n, void* stream) {
    return qx_matvec<Q6KFormat>(x, nullptr, 0.0f, w, y, out_dtype, residual, m, k, n, stream);
}

extern "C" int t2h_q6k_rmsnorm_matvec(const float* h, const float* norm_w, float eps, const void* w, void* y,
                                      int out_dtype, uint32_t k, uint32_t n, void* stream) {
    if (!norm_w) return T2H_ERR_NULL;
    return qx_matvec<Q6KFormat>(h, norm_w, eps, w, y, out_dtype, nullptr, 1, k, n, stream);
}

extern "C" int t2h_q8_0_matvec(const void* x, const void* w, void* y, int out_dtype, const float* residual,
                               uint32_t m, uint32_t k, uint32_t n, void* stream) {
    return qx_matvec<Q80Format>(x, nullptr, 0.0f, w, y, out_dtype, residual, m, k, n, stream);
}

extern "C" int t2h_q6k_lm_head_argmax_partial(const void* x, const float* norm_w, float eps, const void* w,
                                              uint32_t k, uint32_t n, float* partial_scores,
                                              uint32_t* partial_tokens, uint32_t num_partials, void* stream) {
    if (!x || !w || !partial_scores || !partial_tokens) return T2H_ERR_NULL;
    if (num_partials == 0) return T2H_ERR_ARG;
    QxGeom g;
    int st = qx_geometry<Q6KFormat>(k, g);
    if (st) return st;
    if (n == 0) return T2H_ERR_SHAPE;
    QxArgs a = {};
    a.x = x;
    a.norm_w = norm_w;
    a.eps = eps;
    a.w = reinterpret_cast<const uint8_t*>(w);
    a.k = k;
    a.partial_scores = partial_scores;
    a.partial_tokens = partial_tokens;
    return qx_run<Q6KFormat>(norm_w ? QXPRO_RMSNORM : QXPRO_BF16, QXEPI_ARGMAX, a, g, n, num_partials,
                             reinterpret_cast<hipStream_t>(stream));
}
