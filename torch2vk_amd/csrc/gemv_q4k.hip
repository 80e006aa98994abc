// Q4_K dequant-GEMV family for decode (M = 1 token), gfx950.
//
// Replaces the reference's matvec shaders:
//   LINEAR_NOBIAS_Q4_K_MATVEC_F32       (src/models/optimized_qwen3/shaders/linear_nobias_q4_k_matvec_f32.py:26-197)
//   LINEAR_NOBIAS_Q4_K_MATVEC_ADD_F32   (src/models/optimized_qwen3/shaders/linear_nobias_q4_k_matvec_add_f32.py:23-100)
//   LINEAR_NOBIAS_Q4_K_QKV_MATVEC_F32   (src/models/optimized_qwen3/shaders/linear_nobias_q4_k_qkv_matvec_f32.py:22-430)
//   LINEAR_NOBIAS_Q4_K_QK_MATVEC_F32    (src/models/optimized_qwen3/shaders/linear_nobias_q4_k_qk_matvec_f32.py:22-315)
//   + RMS_NORM_MUL_F16_F32 fused as a prologue, SWIGLU_F16 fused as an epilogue,
//   + LM_HEAD_*_ARGMAX_PARTIAL fused as an argmax epilogue.
//
// Weight layout: GGUF Q4_K rows, 144 B per 256-value superblock
// (fp16 d | fp16 dmin | 12 B 6-bit scale/min codes | 128 B nibbles).
//
// Work mapping.  A wave streams 16 superblocks per step: lanes 4s..4s+3 own
// superblock s, and lane l reads the 16-B header plus the 32-B nibble group
// g = l & 3, i.e. all 32 values of sub-block 2g (low nibbles) and of
// sub-block 2g+1 (high nibbles).  One header decode therefore serves 64
// weights.  A "row group" is RPW consecutive rows covered by NIT such steps,
// RPW = 16/gcd(NSB,16) and NIT = NSB*RPW/16, so no lane idles for any K.
//
// Arithmetic.  Nibble pairs become bf16 values 128+q with one and-or
// (0x4300 | q), and v_dot2_f32_bf16 accumulates x*(128+q) in fp32; the 128*Σx
// offset is removed with the per-lane Σx the min term needs anyway:
//   Σ x*w = d*(sc_lo*(S_lo - 128 Σx_lo) + sc_hi*(S_hi - 128 Σx_hi)) - dmin*(m_lo Σx_lo + m_hi Σx_hi)
// x is the same for every row, so each lane keeps its x slice in registers
// for the whole launch; the weight stream is software pipelined.
#include "common.h"

namespace t2h {

enum Q4Prologue { Q4PRO_BF16 = 0, Q4PRO_RMSNORM = 1 };
enum Q4Epilogue { Q4EPI_F32 = 0, Q4EPI_BF16 = 1, Q4EPI_RESID = 2, Q4EPI_SWIGLU = 3, Q4EPI_ARGMAX = 4 };

struct Q4Part {
    const uint8_t* w;
    void* y;
    uint32_t row_begin;
    uint32_t n;
};

struct Q4GemvArgs {
    const void* x;          // Q4PRO_BF16: bf16 [K];  Q4PRO_RMSNORM: fp32 [K]
    const float* norm_w;    // Q4PRO_RMSNORM: fp32 [K]
    const float* residual;  // Q4EPI_RESID: fp32 [N] (may alias y)
    Q4Part parts[3];
    uint32_t n_parts;
    uint32_t n_units;       // row groups (Q4EPI_SWIGLU: row groups of the gate)
    uint32_t units_per_wave;  // every wave runs this many units (rounded up to the ring size, clamped)
    float* partial_scores;  // Q4EPI_ARGMAX: [gridDim.x]
    uint32_t* partial_tokens;
    float eps;
};

constexpr int cgcd(int a, int b) { return b == 0 ? a : cgcd(b, a % b); }

constexpr int GEMV_THREADS = 512;  // 8 waves per block share one staged copy of x
constexpr uint32_t GEMV_WAVES = GEMV_THREADS / 64;

template <int NSB>
struct Q4Geom {
    static constexpr int K = NSB * 256;
    static constexpr int RPW = 16 / cgcd(NSB, 16);
    static constexpr int NIT = NSB * RPW / 16;
    static constexpr int ROW_BYTES = NSB * 144;
};

// Per-lane x slice for one step: the 32 values of sub-block 2g and the 32 of
// sub-block 2g+1, stored as bf16 pairs (e0,e2),(e1,e3),(e4,e6),... to match
// the nibble pairs the and-or trick produces, plus their sums.
struct XSlice {
    uint32_t lo[16];
    uint32_t hi[16];
    float sum_lo;
    float sum_hi;
};

// 32 bf16 values (16 dwords, natural order) -> 16 pairs + their sum
__device__ __forceinline__ void pair_up(const uint32_t (&raw)[16], uint32_t (&out)[16], float& sum) {
    float s = 0.0f;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
        const uint32_t x0 = raw[2 * c];      // (e0, e1)
        const uint32_t x1 = raw[2 * c + 1];  // (e2, e3)
        out[2 * c] = (x0 & 0xffffu) | (x1 << 16);
        out[2 * c + 1] = (x0 >> 16) | (x1 & 0xffff0000u);
        s += bf16_bits_to_f32(x0 & 0xffffu) + bf16_bits_to_f32(x0 >> 16);
        s += bf16_bits_to_f32(x1 & 0xffffu) + bf16_bits_to_f32(x1 >> 16);
    }
    sum = s;
}

__device__ __forceinline__ void unpack_u4x4(const uint4 (&v)[4], uint32_t (&raw)[16]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        raw[4 * i] = v[i].x;
        raw[4 * i + 1] = v[i].y;
        raw[4 * i + 2] = v[i].z;
        raw[4 * i + 3] = v[i].w;
    }
}

// x slice of nibble group g starting at element off (= 64 g within a superblock)
__device__ __forceinline__ void load_xslice(const uint16_t* xb, int off, XSlice& xs) {
    uint4 v[4];
    uint32_t raw[16];
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = load_u4(xb + off + 8 * i);
    unpack_u4x4(v, raw);
    pair_up(raw, xs.lo, xs.sum_lo);
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = load_u4(xb + off + 32 + 8 * i);
    unpack_u4x4(v, raw);
    pair_up(raw, xs.hi, xs.sum_hi);
}

__device__ __forceinline__ void dot_nibble_word(uint32_t w, uint32_t xa, uint32_t xb, uint32_t xc, uint32_t xd,
                                                float& s_lo, float& s_hi) {
    const uint32_t w4 = w >> 4;
    const uint32_t pa = (w & 0x000f000fu) | 0x43004300u;
    const uint32_t pb = ((w >> 8) & 0x000f000fu) | 0x43004300u;
    const uint32_t pc = (w4 & 0x000f000fu) | 0x43004300u;
    const uint32_t pd = ((w4 >> 8) & 0x000f000fu) | 0x43004300u;
    s_lo = dot2_bf16(pa, xa, s_lo);
    s_lo = dot2_bf16(pb, xb, s_lo);
    s_hi = dot2_bf16(pc, xc, s_hi);
    s_hi = dot2_bf16(pd, xd, s_hi);
}

// Partial dot of one lane's 64 values of one superblock (nibble group g).
__device__ __forceinline__ float q4k_lane_dot(const uint4 hdr, const uint4 q0, const uint4 q1, const XSlice& xs,
                                              int g) {
    const float d = f16_bits_to_f32(hdr.x & 0xffffu);
    const float dmin = f16_bits_to_f32(hdr.x >> 16);
    // 6-bit scale/min codes of sub-blocks 2g and 2g+1 (two bytes each)
    const int sh = (g & 1) << 4;
    const bool low = g < 2;
    const uint32_t mask_lo = low ? 0x3f3fu : 0x0f0fu;
    const uint32_t hi_en = low ? 0u : 0x3030u;
    const uint32_t src_s = low ? hdr.y : hdr.w;
    const uint32_t src_m = low ? hdr.z : hdr.w;
    const int sh_m = low ? sh : sh + 4;
    const uint32_t S = ((src_s >> sh) & mask_lo) | ((hdr.y >> (sh + 2)) & hi_en);
    const uint32_t M = ((src_m >> sh_m) & mask_lo) | ((hdr.z >> (sh + 2)) & hi_en);
    const float sc_lo = (float)(S & 0xffu);
    const float sc_hi = (float)((S >> 8) & 0xffu);
    const float m_lo = (float)(M & 0xffu);
    const float m_hi = (float)((M >> 8) & 0xffu);

    float s_lo = 0.0f, s_hi = 0.0f;
    const uint32_t q[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
#pragma unroll
    for (int c = 0; c < 8; ++c)
        dot_nibble_word(q[c], xs.lo[2 * c], xs.lo[2 * c + 1], xs.hi[2 * c], xs.hi[2 * c + 1], s_lo, s_hi);
    const float xq_lo = fmaf(-128.0f, xs.sum_lo, s_lo);
    const float xq_hi = fmaf(-128.0f, xs.sum_hi, s_hi);
    const float scaled = fmaf(sc_lo, xq_lo, sc_hi * xq_hi);
    const float mins = fmaf(m_lo, xs.sum_lo, m_hi * xs.sum_hi);
    return fmaf(d, scaled, -dmin * mins);
}

__device__ __forceinline__ float silu(float g) { return g / (1.0f + expf(-g)); }

template <int NSB, int PRO, int EPI>
__global__ __launch_bounds__(GEMV_THREADS) void q4k_gemv_kernel(const Q4GemvArgs a) {
    using Geo = Q4Geom<NSB>;
    constexpr int K = Geo::K;
    constexpr int RPW = Geo::RPW;
    constexpr int NIT = Geo::NIT;
    constexpr int ROW_BYTES = Geo::ROW_BYTES;
    constexpr int NG = EPI == Q4EPI_SWIGLU ? 2 : 1;  // row groups per unit (gate and up)

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform, scalar
    const int waves_per_block = blockDim.x >> 6;
    const int sbo = lane >> 2;  // superblock slot of this lane within a step
    const int g = lane & 3;     // nibble group: sub-blocks 2g (low nibbles) and 2g+1 (high)

    int rloc[NIT];
    int sbi[NIT];
#pragma unroll
    for (int it = 0; it < NIT; ++it) {
        const int f = it * 16 + sbo;
        rloc[it] = f / NSB;
        sbi[it] = f % NSB;
    }

    // Weight stream, software pipelined over a ring of NSTAGE stages: a stage
    // holds the header and nibble chunks of one unit (NG row groups) and
    // NSTAGE-1 units are in flight while one is reduced.  Every wave runs the
    // same number of units; units past the end are clamped to the last one and
    // their results dropped, so the load stream has no divergent branches.
    constexpr int NSTAGE = (NG * NIT <= 2) ? 3 : 2;
    struct Stage {
        uint4 hdr[NG][NIT];
        uint4 q0[NG][NIT];
        uint4 q1[NG][NIT];
    };
    auto issue = [&](uint32_t unit, Stage& st) {
#pragma unroll
        for (int gi = 0; gi < NG; ++gi) {
#pragma unroll
            for (int it = 0; it < NIT; ++it) {
                const uint8_t* base;
                if constexpr (EPI == Q4EPI_SWIGLU) {
                    const uint32_t row = unit * RPW + (uint32_t)rloc[it];
                    base = a.parts[gi].w + (size_t)row * ROW_BYTES;
                } else {
                    const uint32_t row = unit * RPW + (uint32_t)rloc[it];
                    int pi = 0;
                    pi += (a.n_parts > 1 && row >= a.parts[1].row_begin) ? 1 : 0;
                    pi += (a.n_parts > 2 && row >= a.parts[2].row_begin) ? 1 : 0;
                    const Q4Part& p = a.parts[pi];
                    base = p.w + (size_t)(row - p.row_begin) * ROW_BYTES;
                }
                base += (size_t)sbi[it] * 144;
                st.hdr[gi][it] = load_u4(base);
                // plain (temporal) loads: the two 16-B chunks of a lane are 32 B
                // apart, so each instruction uses half of every line it touches
                // and the other half must still be cached for the next one;
                // non-temporal loads measured ~25% slower here
                st.q0[gi][it] = load_u4(base + 16 + g * 32);
                st.q1[gi][it] = load_u4(base + 32 + g * 32);
            }
        }
    };

    const uint32_t wave_global = blockIdx.x * waves_per_block + wave;
    const uint32_t total_waves = gridDim.x * waves_per_block;
    const uint32_t last_unit = a.n_units - 1;
    auto clamp_unit = [&](uint32_t u) { return u < a.n_units ? u : last_unit; };
    const uint32_t n_iter = (a.units_per_wave + NSTAGE - 1) / NSTAGE * NSTAGE;
    Stage st[NSTAGE];

    // ---------------------------------------------------------- x slice --
    // x is staged once per block in LDS (bf16, coalesced loads shared by the
    // block's waves) and each lane then reads its slices from LDS.  The x-side
    // loads are issued before the first weight stages: vmcnt retires in order,
    // so the prologue waits for them alone while the weight loads stay in flight.
    __shared__ __align__(16) uint16_t xsh[K];
    if constexpr (PRO == Q4PRO_RMSNORM) {
        // one pass: h and norm weight loaded once, sum of squares reduced over
        // the block, normalised bf16 x written to LDS
        constexpr int PT = (K + 4 * GEMV_THREADS - 1) / (4 * GEMV_THREADS);  // float4s per thread
        __shared__ float red[GEMV_THREADS / 64];
        const float* h = reinterpret_cast<const float*>(a.x);
        float4 hv[PT], wv[PT];
#pragma unroll
        for (int j = 0; j < PT; ++j) {
            const int k = (j * GEMV_THREADS + (int)threadIdx.x) * 4;
            if (K % (4 * GEMV_THREADS) == 0 || k < K) {
                hv[j] = *reinterpret_cast<const float4*>(h + k);
                wv[j] = *reinterpret_cast<const float4*>(a.norm_w + k);
            } else {
                hv[j] = make_float4(0.f, 0.f, 0.f, 0.f);
                wv[j] = hv[j];
            }
        }
#pragma unroll
        for (int s = 0; s + 1 < NSTAGE; ++s) issue(clamp_unit(wave_global + s * total_waves), st[s]);
        float ss = 0.0f;
#pragma unroll
        for (int j = 0; j < PT; ++j) {
            ss = fmaf(hv[j].x, hv[j].x, ss);
            ss = fmaf(hv[j].y, hv[j].y, ss);
            ss = fmaf(hv[j].z, hv[j].z, ss);
            ss = fmaf(hv[j].w, hv[j].w, ss);
        }
        ss = wave_sum(ss);
        if (lane == 0) red[wave] = ss;
        __syncthreads();
        float total = 0.0f;
#pragma unroll
        for (int i = 0; i < GEMV_THREADS / 64; ++i) total += red[i];
        const float inv = 1.0f / sqrtf(total / (float)K + a.eps);
#pragma unroll
        for (int j = 0; j < PT; ++j) {
            const int k = (j * GEMV_THREADS + (int)threadIdx.x) * 4;
            if (K % (4 * GEMV_THREADS) == 0 || k < K) {
                const uint32_t p0 = pack_bf16x2(hv[j].x * inv * wv[j].x, hv[j].y * inv * wv[j].y);
                const uint32_t p1 = pack_bf16x2(hv[j].z * inv * wv[j].z, hv[j].w * inv * wv[j].w);
                *reinterpret_cast<uint2*>(&xsh[k]) = make_uint2(p0, p1);
            }
        }
    } else {
        constexpr int PT = (K + 8 * GEMV_THREADS - 1) / (8 * GEMV_THREADS);  // 16-B chunks per thread
        const uint16_t* xb = reinterpret_cast<const uint16_t*>(a.x);
        uint4 xv[PT];
#pragma unroll
        for (int j = 0; j < PT; ++j) {
            const int k = (j * GEMV_THREADS + (int)threadIdx.x) * 8;
            xv[j] = (K % (8 * GEMV_THREADS) == 0 || k < K) ? load_u4(xb + k) : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int s = 0; s + 1 < NSTAGE; ++s) issue(clamp_unit(wave_global + s * total_waves), st[s]);
#pragma unroll
        for (int j = 0; j < PT; ++j) {
            const int k = (j * GEMV_THREADS + (int)threadIdx.x) * 8;
            if (K % (8 * GEMV_THREADS) == 0 || k < K) *reinterpret_cast<uint4*>(&xsh[k]) = xv[j];
        }
    }
    __syncthreads();
    XSlice xs[NIT];
#pragma unroll
    for (int it = 0; it < NIT; ++it) load_xslice(xsh, sbi[it] * 256 + 64 * g, xs[it]);

    float best_score = -3.4028234663852886e38f;
    uint32_t best_token = 0xffffffffu;

    auto consume = [&](uint32_t u, const Stage& st) {
        const bool live = u < a.n_units;
        float res[NG][RPW];
#pragma unroll
        for (int gi = 0; gi < NG; ++gi) {
            float acc[RPW];
#pragma unroll
            for (int r = 0; r < RPW; ++r) acc[r] = 0.0f;
#pragma unroll
            for (int it = 0; it < NIT; ++it) {
                const float c = q4k_lane_dot(st.hdr[gi][it], st.q0[gi][it], st.q1[gi][it], xs[it], g);
                if constexpr (RPW == 1) {
                    acc[0] += c;
                } else {
#pragma unroll
                    for (int r = 0; r < RPW; ++r) acc[r] += (rloc[it] == r) ? c : 0.0f;
                }
            }
#pragma unroll
            for (int r = 0; r < RPW; ++r) res[gi][r] = wave_sum(acc[r]);
        }
        const uint32_t row0 = u * RPW;
        if (!live) return;
        if constexpr (EPI == Q4EPI_SWIGLU) {
            if (lane < RPW) {
                float gv = res[0][0], uv = res[1][0];
#pragma unroll
                for (int r = 1; r < RPW; ++r) {
                    gv = (lane == r) ? res[0][r] : gv;
                    uv = (lane == r) ? res[1][r] : uv;
                }
                reinterpret_cast<uint16_t*>(a.parts[0].y)[row0 + lane] = (uint16_t)f32_to_bf16_bits(silu(gv) * uv);
            }
        } else if constexpr (EPI == Q4EPI_ARGMAX) {
#pragma unroll
            for (int r = 0; r < RPW; ++r) {
                if (better_pair(res[0][r], row0 + r, best_score, best_token)) {
                    best_score = res[0][r];
                    best_token = row0 + r;
                }
            }
        } else if (lane < RPW) {
            // lane r stores row r of the group (res[] is wave-uniform)
            float v = res[0][0];
#pragma unroll
            for (int r = 1; r < RPW; ++r) v = (lane == r) ? res[0][r] : v;
            const uint32_t row = row0 + lane;
            int pi = 0;
            pi += (a.n_parts > 1 && row >= a.parts[1].row_begin) ? 1 : 0;
            pi += (a.n_parts > 2 && row >= a.parts[2].row_begin) ? 1 : 0;
            const Q4Part& p = a.parts[pi];
            const uint32_t local = row - p.row_begin;
            if constexpr (EPI == Q4EPI_F32) {
                reinterpret_cast<float*>(p.y)[local] = v;
            } else if constexpr (EPI == Q4EPI_BF16) {
                reinterpret_cast<uint16_t*>(p.y)[local] = (uint16_t)f32_to_bf16_bits(v);
            } else if constexpr (EPI == Q4EPI_RESID) {
                reinterpret_cast<float*>(p.y)[local] = a.residual[local] + v;
            }
        }
    };

    // ring over the units of this wave: issue unit i+NSTAGE-1, reduce unit i
    for (uint32_t i = 0; i < n_iter; i += NSTAGE) {
#pragma unroll
        for (int s = 0; s < NSTAGE; ++s) {
            const uint32_t ui = i + s;
            if (ui + NSTAGE - 1 < n_iter)
                issue(clamp_unit(wave_global + (ui + NSTAGE - 1) * total_waves), st[(s + NSTAGE - 1) % NSTAGE]);
            consume(wave_global + ui * total_waves, st[s]);
        }
    }

    if constexpr (EPI == Q4EPI_ARGMAX) {
        __shared__ float bs[16];
        __shared__ uint32_t bt[16];
        if (lane == 0) {
            bs[wave] = best_score;
            bt[wave] = best_token;
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            float s = bs[0];
            uint32_t t = bt[0];
            for (int i = 1; i < waves_per_block; ++i) {
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

template <int PRO, int EPI>
static hipError_t launch_nsb(uint32_t nsb, dim3 grid, dim3 block, const Q4GemvArgs& a, hipStream_t s) {
    switch (nsb) {
#define T2H_Q4_CASE(N)                                                                      \
    case N:                                                                                 \
        hipLaunchKernelGGL((q4k_gemv_kernel<N, PRO, EPI>), grid, block, 0, s, a); \
        return hipGetLastError();
        T2H_Q4_CASE(1)
        T2H_Q4_CASE(2)
        T2H_Q4_CASE(3)
        T2H_Q4_CASE(4)
        T2H_Q4_CASE(8)
        T2H_Q4_CASE(12)
        T2H_Q4_CASE(16)
        T2H_Q4_CASE(24)
        T2H_Q4_CASE(32)
        T2H_Q4_CASE(48)
#undef T2H_Q4_CASE
        default:
            return hipErrorInvalidValue;
    }
}

static bool nsb_supported(uint32_t nsb) {
    switch (nsb) {
        case 1: case 2: case 3: case 4: case 8: case 12: case 16: case 24: case 32: case 48:
            return true;
        default:
            return false;
    }
}

static uint32_t rows_per_group(uint32_t nsb) {
    uint32_t a = nsb, b = 16;
    while (b) {
        const uint32_t t = a % b;
        a = b;
        b = t;
    }
    return 16u / a;
}

// Grid: enough blocks of 4 waves that every wave gets about `units_per_wave`
// row groups, capped so that the launch stays a few blocks per CU.
static uint32_t units_per_wave(uint32_t n_units, uint32_t blocks) {
    const uint32_t waves = blocks * GEMV_WAVES;
    return (n_units + waves - 1u) / waves;
}

static uint32_t pick_blocks(uint32_t n_units, uint32_t max_blocks) {
    if (max_blocks == 0) max_blocks = 1;
    const uint32_t u = units_per_wave(n_units, max_blocks);
    uint32_t blocks = (n_units + GEMV_WAVES * u - 1u) / (GEMV_WAVES * u);
    if (blocks == 0) blocks = 1;
    return blocks;
}

static uint32_t g_max_blocks = 256;        // blocks of GEMV_WAVES waves, plain x input
static uint32_t g_max_blocks_norm = 256;   // RMSNorm prologue: each block re-reads h and the norm weight

}  // namespace t2h

using namespace t2h;

static int validate_q4(uint32_t k) {
    if (k == 0 || k % 256 != 0) return T2H_ERR_SHAPE;
    if (!nsb_supported(k / 256)) return T2H_ERR_UNSUPPORTED;
    return T2H_OK;
}

extern "C" int t2h_set_gemv_max_blocks(uint32_t max_blocks, uint32_t max_blocks_norm) {
    if (max_blocks == 0) return T2H_ERR_ARG;
    g_max_blocks = max_blocks;
    g_max_blocks_norm = max_blocks_norm ? max_blocks_norm : max_blocks;
    return T2H_OK;
}

static int q4k_launch(int pro, int epi, Q4GemvArgs a, uint32_t nsb, uint32_t blocks, hipStream_t s) {
    if (a.n_units == 0) return T2H_OK;
    a.units_per_wave = units_per_wave(a.n_units, blocks);
    const dim3 grid(blocks), block(GEMV_THREADS);
    hipError_t e = hipErrorInvalidValue;
    if (pro == Q4PRO_BF16) {
        switch (epi) {
            case Q4EPI_F32: e = launch_nsb<Q4PRO_BF16, Q4EPI_F32>(nsb, grid, block, a, s); break;
            case Q4EPI_BF16: e = launch_nsb<Q4PRO_BF16, Q4EPI_BF16>(nsb, grid, block, a, s); break;
            case Q4EPI_RESID: e = launch_nsb<Q4PRO_BF16, Q4EPI_RESID>(nsb, grid, block, a, s); break;
            case Q4EPI_ARGMAX: e = launch_nsb<Q4PRO_BF16, Q4EPI_ARGMAX>(nsb, grid, block, a, s); break;
            default: return T2H_ERR_ARG;
        }
    } else {
        switch (epi) {
            case Q4EPI_F32: e = launch_nsb<Q4PRO_RMSNORM, Q4EPI_F32>(nsb, grid, block, a, s); break;
            case Q4EPI_SWIGLU: e = launch_nsb<Q4PRO_RMSNORM, Q4EPI_SWIGLU>(nsb, grid, block, a, s); break;
            case Q4EPI_ARGMAX: e = launch_nsb<Q4PRO_RMSNORM, Q4EPI_ARGMAX>(nsb, grid, block, a, s); break;
            default: return T2H_ERR_ARG;
        }
    }
    return e == hipSuccess ? T2H_OK : T2H_ERR_HIP_BASE + (int)e;
}

static int fill_parts(Q4GemvArgs& a, uint32_t n_parts, const void* const* w, void* const* y, const uint32_t* n,
                      uint32_t rpw, uint32_t* total) {
    if (n_parts == 0 || n_parts > 3 || !w || !n) return T2H_ERR_ARG;
    uint32_t begin = 0;
    for (uint32_t i = 0; i < n_parts; ++i) {
        if (!w[i] || (y && !y[i])) return T2H_ERR_NULL;
        if (n[i] == 0 || n[i] % rpw != 0) return T2H_ERR_SHAPE;
        a.parts[i].w = reinterpret_cast<const uint8_t*>(w[i]);
        a.parts[i].y = y ? y[i] : nullptr;
        a.parts[i].row_begin = begin;
        a.parts[i].n = n[i];
        begin += n[i];
    }
    for (uint32_t i = n_parts; i < 3; ++i) {
        a.parts[i] = a.parts[n_parts - 1];
        a.parts[i].row_begin = 0xffffffffu;
    }
    a.n_parts = n_parts;
    *total = begin;
    return T2H_OK;
}

extern "C" int t2h_q4k_matvec(const void* x, const void* w, void* y, int out_dtype, const float* residual,
                              uint32_t m, uint32_t k, uint32_t n, void* stream) {
    if (!x || !w || !y) return T2H_ERR_NULL;
    int st = validate_q4(k);
    if (st) return st;
    if (m == 0 || n == 0) return T2H_OK;
    const uint32_t nsb = k / 256;
    const uint32_t rpw = rows_per_group(nsb);
    if (n % rpw != 0) return T2H_ERR_SHAPE;
    int epi;
    if (residual) {
        if (out_dtype != T2H_DTYPE_F32) return T2H_ERR_DTYPE;
        epi = Q4EPI_RESID;
    } else if (out_dtype == T2H_DTYPE_F32) {
        epi = Q4EPI_F32;
    } else if (out_dtype == T2H_DTYPE_BF16) {
        epi = Q4EPI_BF16;
    } else {
        return T2H_ERR_DTYPE;
    }
    const size_t out_size = out_dtype == T2H_DTYPE_F32 ? 4 : 2;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    for (uint32_t row = 0; row < m; ++row) {
        Q4GemvArgs a = {};
        const void* wv[1] = {w};
        void* yv[1] = {reinterpret_cast<uint8_t*>(y) + (size_t)row * n * out_size};
        uint32_t total = 0;
        st = fill_parts(a, 1, wv, yv, &n, rpw, &total);
        if (st) return st;
        a.x = reinterpret_cast<const uint16_t*>(x) + (size_t)row * k;
        a.residual = residual ? residual + (size_t)row * n : nullptr;
        a.n_units = total / rpw;
        st = q4k_launch(Q4PRO_BF16, epi, a, nsb, pick_blocks(a.n_units, g_max_blocks), s);
        if (st) return st;
    }
    return T2H_OK;
}

extern "C" int t2h_q4k_matvec_multi(const void* x, const float* norm_w, float eps, uint32_t n_parts,
                                    const void* const* w, void* const* y, const uint32_t* n, uint32_t k,
                                    int out_dtype, void* stream) {
    if (!x || !y) return T2H_ERR_NULL;
    int st = validate_q4(k);
    if (st) return st;
    const uint32_t nsb = k / 256;
    const uint32_t rpw = rows_per_group(nsb);
    Q4GemvArgs a = {};
    uint32_t total = 0;
    st = fill_parts(a, n_parts, w, y, n, rpw, &total);
    if (st) return st;
    a.x = x;
    a.norm_w = norm_w;
    a.eps = eps;
    a.n_units = total / rpw;
    int pro = norm_w ? Q4PRO_RMSNORM : Q4PRO_BF16;
    int epi;
    if (out_dtype == T2H_DTYPE_F32) {
        epi = Q4EPI_F32;
    } else if (out_dtype == T2H_DTYPE_BF16 && !norm_w) {
        epi = Q4EPI_BF16;
    } else {
        return T2H_ERR_DTYPE;
    }
    return q4k_launch(pro, epi, a, nsb, pick_blocks(a.n_units, norm_w ? g_max_blocks_norm : g_max_blocks),
                      reinterpret_cast<hipStream_t>(stream));
}

extern "C" int t2h_q4k_rmsnorm_swiglu_matvec(const float* h, const float* norm_w, float eps, const void* w_gate,
                                             const void* w_up, void* act_out, uint32_t k, uint32_t n,
                                             void* stream) {
    if (!h || !norm_w || !w_gate || !w_up || !act_out) return T2H_ERR_NULL;
    int st = validate_q4(k);
    if (st) return st;
    const uint32_t nsb = k / 256;
    const uint32_t rpw = rows_per_group(nsb);
    Q4GemvArgs a = {};
    const void* wv[2] = {w_gate, w_up};
    void* yv[2] = {act_out, act_out};
    const uint32_t nv[2] = {n, n};
    uint32_t total = 0;
    st = fill_parts(a, 2, wv, yv, nv, rpw, &total);
    if (st) return st;
    a.x = h;
    a.norm_w = norm_w;
    a.eps = eps;
    a.n_units = n / rpw;
    return q4k_launch(Q4PRO_RMSNORM, Q4EPI_SWIGLU, a, nsb, pick_blocks(a.n_units, g_max_blocks_norm),
                      reinterpret_cast<hipStream_t>(stream));
}

extern "C" int t2h_q4k_lm_head_argmax_partial(const void* x, const float* norm_w, float eps, const void* w,
                                              uint32_t k, uint32_t n, float* partial_scores,
                                              uint32_t* partial_tokens, uint32_t num_partials, void* stream) {
    if (!x || !w || !partial_scores || !partial_tokens) return T2H_ERR_NULL;
    int st = validate_q4(k);
    if (st) return st;
    const uint32_t nsb = k / 256;
    const uint32_t rpw = rows_per_group(nsb);
    if (num_partials == 0) return T2H_ERR_ARG;
    Q4GemvArgs a = {};
    const void* wv[1] = {w};
    uint32_t total = 0;
    st = fill_parts(a, 1, wv, nullptr, &n, rpw, &total);
    if (st) return st;
    a.x = x;
    a.norm_w = norm_w;
    a.eps = eps;
    a.n_units = n / rpw;
    a.partial_scores = partial_scores;
    a.partial_tokens = partial_tokens;
    return q4k_launch(norm_w ? Q4PRO_RMSNORM : Q4PRO_BF16, Q4EPI_ARGMAX, a, nsb, num_partials,
                      reinterpret_cast<hipStream_t>(stream));
}
