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
// weights.  A "unit" is RPW consecutive rows covered by NIT such steps,
// RPW = 16/gcd(NSBW,16) and NIT = NSBW*RPW/16, where NSBW is the number of
// superblocks a wave covers per row: all NSB of them, or, for rows of 32 or
// 48 superblocks, one 16-superblock chunk, with KS = NSB/16 waves splitting
// each row and adding their partial sums in LDS.  No lane idles for any K.
//
// Arithmetic.  A nibble pair becomes two fp16 operands of v_dot2_f32_f16 with
// one and-or against the fp16 magic 64.0 (0x5400):
//   (w & 0x000f000f) | 0x54005400 = (64 + q/16) x2   (low nibbles)
//   (w & 0x00f000f0) | 0x54005400 = (64 + q)    x2   (high nibbles)
// so 8 nibbles cost 5 bit operations and 4 dot2.  The 64*sum(x) offset comes
// off with the per-sub-block sums of x that the min term needs anyway:
//   sum x*q = 16*(S_lo - 64 sum x_lo)  and  S_hi - 64 sum x_hi.
// Every product is exact in fp32; the offset cancels to a few fp32 ulps of
// 64*sum|x| per sub-block.  x is bf16 by contract and enters the dot as fp16,
// which holds every bf16 value of magnitude 2^-14..65504 exactly (the
// reference's activations are fp16, so its range is the same).  The block
// stages x once in LDS, already as fp16 pair words (e0,e2),(e1,e3) that line
// up with the nibble pairs, plus the sum of every 32-value sub-block; each
// lane then keeps its slices in registers for the whole launch.
#include "q4k_device.h"

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
    uint32_t n_units;         // units of RPW rows (Q4EPI_SWIGLU: units of the gate)
    uint32_t units_per_wave;  // every wave runs this many units (rounded up to the ring size, clamped)
    float* partial_scores;    // Q4EPI_ARGMAX: [gridDim.x]
    uint32_t* partial_tokens;
    float eps;
};

// Units one wave may own when KS > 1 (their partial sums wait in LDS).
constexpr uint32_t Q4_KSPLIT_MAX_UNITS = 8;

template <int NSB, int KS, int WPB, int PRO, int EPI, int UPW = 0>
__global__ __launch_bounds__(WPB * 64) void q4k_gemv_kernel(const Q4GemvArgs a) {
    constexpr int K = NSB * 256;
    constexpr int NT = WPB * 64;
    constexpr int WR = WPB / KS;          // wave rows per block
    constexpr int NSBW = NSB / KS;        // superblocks per wave and row
    constexpr int RPW = 16 / cgcd(NSBW, 16);
    constexpr int NIT = NSBW * RPW / 16;
    constexpr int ROW_BYTES = NSB * 144;
    constexpr int NG = EPI == Q4EPI_SWIGLU ? 2 : 1;  // row groups per unit (gate and up)
    static_assert(WPB % KS == 0 && NSB % KS == 0, "KS must divide the block and the row");
    static_assert(KS == 1 || NSBW == 16, "split rows are cut into 16-superblock chunks");
    static_assert(KS == 1 || (EPI != Q4EPI_SWIGLU && EPI != Q4EPI_ARGMAX), "split rows: plain epilogues only");

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform, scalar
    const int ks = wave % KS;
    const int wr = wave / KS;
    const int sbo = lane >> 2;  // superblock slot of this lane within a step
    const int g = lane & 3;     // nibble group: sub-blocks 2g (low nibbles) and 2g+1 (high)

    int rloc[NIT];
    int sbi[NIT];
#pragma unroll
    for (int it = 0; it < NIT; ++it) {
        const int f = it * 16 + sbo;
        rloc[it] = f / NSBW;
        sbi[it] = ks * NSBW + f % NSBW;
    }

    // Weight stream, software pipelined over a ring of NSTAGE stages: a stage
    // holds the header and nibble chunks of one unit (NG row groups).  The
    // first NSTAGE units are issued before the x prologue; a stage is refilled
    // with unit i+NSTAGE as soon as unit i has been reduced.  Every wave runs
    // the same number of units; units past the end are clamped to the last one
    // and their results dropped, so the load stream has no divergent branches.
    // (gate|up rows of 3 steps per unit hold 72 VGPRs of weights per stage: one stage, so nothing spills)
    constexpr int NSTAGE = UPW > 0 ? UPW : ((NG * NIT == 1) ? 4 : (NG * NIT >= 6 ? 1 : 2));
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
                const uint32_t row = unit * RPW + (uint32_t)rloc[it];
                if constexpr (EPI == Q4EPI_SWIGLU) {
                    base = a.parts[gi].w + (size_t)row * ROW_BYTES;
                } else {
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
                // and the other half must still be cached for the next one
                st.q0[gi][it] = load_u4(base + 16 + g * 32);
                st.q1[gi][it] = load_u4(base + 32 + g * 32);
            }
        }
    };

    const uint32_t wrow = blockIdx.x * WR + wr;
    const uint32_t total_wrows = gridDim.x * WR;
    const uint32_t last_unit = a.n_units - 1;
    auto clamp_unit = [&](uint32_t u) { return u < a.n_units ? u : last_unit; };
    const uint32_t n_iter = UPW > 0 ? (uint32_t)UPW : a.units_per_wave;  // the same for every wave
    Stage st[NSTAGE];

    // ---------------------------------------------------------- x slice --
    // x is staged once per block in LDS (coalesced loads shared by the
    // block's waves) and each lane then reads its slices from LDS.  The x-side
    // loads go first and only the first weight stage is issued before the
    // prologue: vmcnt retires in order, so the prologue waits for x alone.
    __shared__ __align__(16) uint32_t xp[xp_words(K)];
    __shared__ float xsum[K / 32];
    constexpr int PT = (K + 4 * NT - 1) / (4 * NT);  // 4-value groups per thread
    if constexpr (PRO == Q4PRO_RMSNORM) {
        // one pass: h and norm weight loaded once, sum of squares reduced over
        // the block, normalised x (rounded to bf16) staged in LDS
        __shared__ float red[WPB];
        const float* h = reinterpret_cast<const float*>(a.x);
        float4 hv[PT], wv[PT];
#pragma unroll
        for (int j = 0; j < PT; ++j) {
            const int k = (j * NT + (int)threadIdx.x) * 4;
            if (K % (4 * NT) == 0 || k < K) {
                hv[j] = *reinterpret_cast<const float4*>(h + k);
                wv[j] = *reinterpret_cast<const float4*>(a.norm_w + k);
            } else {
                hv[j] = make_float4(0.f, 0.f, 0.f, 0.f);
                wv[j] = hv[j];
            }
        }
        issue(clamp_unit(wrow), st[0]);
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
        for (int i = 0; i < WPB; ++i) total += red[i];
        const float inv = 1.0f / sqrtf(total / (float)K + a.eps);
#pragma unroll
        for (int j = 0; j < PT; ++j) {
            const int k = (j * NT + (int)threadIdx.x) * 4;
            if (K % (4 * NT) == 0 || k < K)
                stage_x4(xp, xsum, k, bf16_round(hv[j].x * inv * wv[j].x), bf16_round(hv[j].y * inv * wv[j].y),
                         bf16_round(hv[j].z * inv * wv[j].z), bf16_round(hv[j].w * inv * wv[j].w));
        }
    } else {
        const uint16_t* xb = reinterpret_cast<const uint16_t*>(a.x);
        uint2 xv[PT];
#pragma unroll
        for (int j = 0; j < PT; ++j) {
            const int k = (j * NT + (int)threadIdx.x) * 4;
            xv[j] = (K % (4 * NT) == 0 || k < K) ? *reinterpret_cast<const uint2*>(xb + k) : make_uint2(0, 0);
        }
        issue(clamp_unit(wrow), st[0]);
#pragma unroll
        for (int j = 0; j < PT; ++j) {
            const int k = (j * NT + (int)threadIdx.x) * 4;
            if (K % (4 * NT) == 0 || k < K)
                stage_x4(xp, xsum, k, bf16_bits_to_f32(xv[j].x & 0xffffu), bf16_bits_to_f32(xv[j].x >> 16),
                         bf16_bits_to_f32(xv[j].y & 0xffffu), bf16_bits_to_f32(xv[j].y >> 16));
        }
    }
    __syncthreads();
    // The other stages are issued only now: a wave's loads return in order and
    // the CU's memory pipeline is shared, so x-side loads queued behind a deep
    // weight stream would hold the whole block at the barrier above.
#pragma unroll
    for (int s = 1; s < NSTAGE; ++s)
        if ((uint32_t)s < n_iter) issue(clamp_unit(wrow + s * total_wrows), st[s]);
    // A lane's x slices (34 VGPRs per step) stay in registers for the whole launch when they fit beside the
    // weight ring; otherwise (3 steps per unit, or gate|up rings of 2 steps) each unit re-reads them from LDS,
    // which keeps the kernel within 256 VGPRs without scratch.
    constexpr bool XREG = NIT * 34 + NSTAGE * NG * NIT * 12 <= 160;
    XSlice16 xs[XREG ? NIT : 1];
    if constexpr (XREG) {
#pragma unroll
        for (int it = 0; it < NIT; ++it) load_xslice16(xp, xsum, sbi[it], g, xs[it]);
    }
    const Q4LaneConsts lc = q4k_lane_consts(g);

    float best_score = -3.4028234663852886e38f;
    uint32_t best_token = 0xffffffffu;

    auto store_row = [&](uint32_t row, float v) {
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
    };

    constexpr int PART_WR = KS > 1 ? WR : 1;
    constexpr int PART_KS = KS > 1 ? KS : 1;
    constexpr int PART_U = KS > 1 ? (int)Q4_KSPLIT_MAX_UNITS : 1;
    __shared__ float part[PART_WR][PART_U][PART_KS];

    auto consume = [&](uint32_t i, uint32_t u, const Stage& st) {
        const bool live = u < a.n_units;
        float acc[NG][RPW];
#pragma unroll
        for (int gi = 0; gi < NG; ++gi) {
#pragma unroll
            for (int r = 0; r < RPW; ++r) acc[gi][r] = 0.0f;
        }
#pragma unroll
        for (int it = 0; it < NIT; ++it) {
            XSlice16 xl;
            if constexpr (!XREG) load_xslice16(xp, xsum, sbi[it], g, xl);
            const XSlice16& x = XREG ? xs[XREG ? it : 0] : xl;
#pragma unroll
            for (int gi = 0; gi < NG; ++gi) {
                const float c = q4k_lane_dot(st.hdr[gi][it], st.q0[gi][it], st.q1[gi][it], x, lc);
                if constexpr (RPW == 1) {
                    acc[gi][0] += c;
                } else {
#pragma unroll
                    for (int r = 0; r < RPW; ++r) acc[gi][r] += (rloc[it] == r) ? c : 0.0f;
                }
            }
        }
        float res[NG][RPW];
#pragma unroll
        for (int gi = 0; gi < NG; ++gi) {
#pragma unroll
            for (int r = 0; r < RPW; ++r) res[gi][r] = wave_sum(acc[gi][r]);
        }
        const uint32_t row0 = u * RPW;
        if (!live) return;
        if constexpr (KS > 1) {
            // partial of chunk ks; the block adds the KS chunks after the loop
            if (lane == 0) part[wr][i][ks] = res[0][0];
        } else if constexpr (EPI == Q4EPI_SWIGLU) {
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
            // lane r stores row r of the unit (res[] is wave-uniform)
            float v = res[0][0];
#pragma unroll
            for (int r = 1; r < RPW; ++r) v = (lane == r) ? res[0][r] : v;
            store_row(row0 + lane, v);
        }
    };

    if constexpr (UPW > 0) {
        // every unit was issued up front: reduce them in order, no loop
#pragma unroll
        for (int s = 0; s < UPW; ++s) consume(s, wrow + s * total_wrows, st[s]);
    } else
    // ring over the units of this wave: reduce unit i, refill its stage with unit i+NSTAGE
    for (uint32_t i = 0; i < n_iter; i += NSTAGE) {
#pragma unroll
        for (int s = 0; s < NSTAGE; ++s) {
            const uint32_t ui = i + s;
            if (ui >= n_iter) break;  // wave-uniform
            consume(ui, wrow + ui * total_wrows, st[s]);
            if (ui + NSTAGE < n_iter) issue(clamp_unit(wrow + (ui + NSTAGE) * total_wrows), st[s]);
        }
    }

    if constexpr (KS > 1) {
        __syncthreads();
        const uint32_t t = threadIdx.x;
        if (t < (uint32_t)WR * a.units_per_wave) {
            const uint32_t w = t / a.units_per_wave, i = t % a.units_per_wave;
            const uint32_t u = (blockIdx.x * WR + w) + i * total_wrows;
            if (u < a.n_units) {
                float v = 0.0f;
#pragma unroll
                for (int k2 = 0; k2 < KS; ++k2) v += part[w][i][k2];
                store_row(u, v);
            }
        }
    }

    if constexpr (EPI == Q4EPI_ARGMAX) {
        __shared__ float bs[WPB];
        __shared__ uint32_t bt[WPB];
        if (lane == 0) {
            bs[wave] = best_score;
            bt[wave] = best_token;
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            float s = bs[0];
            uint32_t t = bt[0];
            for (int i = 1; i < WPB; ++i) {
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

// Launch geometry of one row length: KS waves split each row when it is 32
// or 48 superblocks long and the epilogue allows it; blocks hold WPB waves.
struct Q4Geometry {
    uint32_t ks;
    uint32_t wpb;
    uint32_t rpw;  // rows per unit
    uint32_t wr() const { return wpb / ks; }
};

static uint32_t gcd_u32(uint32_t a, uint32_t b) {
    while (b) {
        const uint32_t t = a % b;
        a = b;
        b = t;
    }
    return a;
}

static bool nsb_supported(uint32_t nsb) {
    switch (nsb) {
        case 1: case 2: case 3: case 4: case 8: case 12: case 16: case 24: case 32: case 48:
            return true;
        default:
            return false;
    }
}

static Q4Geometry q4_geometry(uint32_t nsb, int epi) {
    Q4Geometry g;
    const bool splittable = epi != Q4EPI_SWIGLU && epi != Q4EPI_ARGMAX;
    g.ks = (splittable && (nsb == 32 || nsb == 48)) ? nsb / 16 : 1;
    g.wpb = g.ks == 3 ? 12 : 8;
    g.rpw = 16u / gcd_u32(nsb / g.ks, 16);
    return g;
}

// Row lengths with straight-line kernels for 1..4 units per wave (the decode
// shapes of Qwen3-0.6B and -8B); every other launch runs the ring loop.
static bool q4_straight_line(uint32_t nsb, int epi) {
    return epi != Q4EPI_ARGMAX && (nsb == 4 || nsb == 16 || (nsb == 48 && epi != Q4EPI_SWIGLU));
}

template <int NSB, int KS, int WPB, int PRO, int EPI>
static void launch_upw(uint32_t upw, dim3 grid, const Q4GemvArgs& a, hipStream_t s) {
    const dim3 block(WPB * 64);
    if constexpr (EPI != Q4EPI_ARGMAX && (NSB == 4 || NSB == 16 || (NSB == 48 && EPI != Q4EPI_SWIGLU))) {
        switch (upw) {
            case 1: hipLaunchKernelGGL((q4k_gemv_kernel<NSB, KS, WPB, PRO, EPI, 1>), grid, block, 0, s, a); return;
            case 2: hipLaunchKernelGGL((q4k_gemv_kernel<NSB, KS, WPB, PRO, EPI, 2>), grid, block, 0, s, a); return;
            case 3: hipLaunchKernelGGL((q4k_gemv_kernel<NSB, KS, WPB, PRO, EPI, 3>), grid, block, 0, s, a); return;
            case 4: hipLaunchKernelGGL((q4k_gemv_kernel<NSB, KS, WPB, PRO, EPI, 4>), grid, block, 0, s, a); return;
            default: break;
        }
    }
    hipLaunchKernelGGL((q4k_gemv_kernel<NSB, KS, WPB, PRO, EPI, 0>), grid, block, 0, s, a);
}

template <int PRO, int EPI>
static hipError_t launch_nsb(uint32_t nsb, uint32_t ks, uint32_t upw, dim3 grid, const Q4GemvArgs& a,
                             hipStream_t s) {
    switch (nsb) {
        case 1: launch_upw<1, 1, 8, PRO, EPI>(0, grid, a, s); break;
        case 2: launch_upw<2, 1, 8, PRO, EPI>(0, grid, a, s); break;
        case 3: launch_upw<3, 1, 8, PRO, EPI>(0, grid, a, s); break;
        case 4: launch_upw<4, 1, 8, PRO, EPI>(upw, grid, a, s); break;
        case 8: launch_upw<8, 1, 8, PRO, EPI>(0, grid, a, s); break;
        case 12: launch_upw<12, 1, 8, PRO, EPI>(0, grid, a, s); break;
        case 16: launch_upw<16, 1, 8, PRO, EPI>(upw, grid, a, s); break;
        case 24: launch_upw<24, 1, 8, PRO, EPI>(0, grid, a, s); break;
        case 32:
            if constexpr (EPI == Q4EPI_SWIGLU || EPI == Q4EPI_ARGMAX) launch_upw<32, 1, 8, PRO, EPI>(0, grid, a, s);
            else if (ks == 2) launch_upw<32, 2, 8, PRO, EPI>(0, grid, a, s);
            else return hipErrorInvalidValue;
            break;
        case 48:
            if constexpr (EPI == Q4EPI_SWIGLU || EPI == Q4EPI_ARGMAX) launch_upw<48, 1, 8, PRO, EPI>(0, grid, a, s);
            else if (ks == 3) launch_upw<48, 3, 12, PRO, EPI>(upw, grid, a, s);
            else return hipErrorInvalidValue;
            break;
        default:
            return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// Grid: wave rows of `units_per_wave` units each, at most `max_blocks` blocks
// (more when a split-row launch caps its units per wave).
static uint32_t units_per_wave_for(uint32_t n_units, uint32_t blocks, const Q4Geometry& g) {
    const uint32_t wrows = blocks * g.wr();
    uint32_t u = (n_units + wrows - 1u) / wrows;
    if (g.ks > 1 && u > Q4_KSPLIT_MAX_UNITS) u = Q4_KSPLIT_MAX_UNITS;
    return u ? u : 1u;
}

static uint32_t blocks_for(uint32_t n_units, uint32_t upw, const Q4Geometry& g) {
    const uint32_t per_block = g.wr() * upw;
    const uint32_t b = (n_units + per_block - 1u) / per_block;
    return b ? b : 1u;
}

// Grid caps in blocks (tuned on MI355X at the Qwen3-8B decode shapes).
static uint32_t g_max_blocks = 256;       // plain bf16 x
static uint32_t g_max_blocks_norm = 256;  // fused RMSNorm prologue

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

// Launch over `max_blocks` (or exactly `fixed_blocks` blocks when non-zero).
static int q4k_launch(int pro, int epi, Q4GemvArgs a, uint32_t nsb, uint32_t max_blocks, uint32_t fixed_blocks,
                      hipStream_t s) {
    if (a.n_units == 0) return T2H_OK;
    const Q4Geometry geo = q4_geometry(nsb, epi);
    uint32_t blocks;
    if (fixed_blocks) {
        blocks = fixed_blocks;
        a.units_per_wave = units_per_wave_for(a.n_units, blocks, geo);
        if (blocks_for(a.n_units, a.units_per_wave, geo) > blocks) return T2H_ERR_ARG;
    } else {
        a.units_per_wave = units_per_wave_for(a.n_units, max_blocks ? max_blocks : 1u, geo);
        blocks = blocks_for(a.n_units, a.units_per_wave, geo);
    }
    const dim3 grid(blocks);
    const uint32_t upw = q4_straight_line(nsb, epi) && a.units_per_wave <= 4 ? a.units_per_wave : 0;
    hipError_t e = hipErrorInvalidValue;
    if (pro == Q4PRO_BF16) {
        switch (epi) {
            case Q4EPI_F32: e = launch_nsb<Q4PRO_BF16, Q4EPI_F32>(nsb, geo.ks, upw, grid, a, s); break;
            case Q4EPI_BF16: e = launch_nsb<Q4PRO_BF16, Q4EPI_BF16>(nsb, geo.ks, upw, grid, a, s); break;
            case Q4EPI_RESID: e = launch_nsb<Q4PRO_BF16, Q4EPI_RESID>(nsb, geo.ks, upw, grid, a, s); break;
            case Q4EPI_ARGMAX: e = launch_nsb<Q4PRO_BF16, Q4EPI_ARGMAX>(nsb, geo.ks, upw, grid, a, s); break;
            default: return T2H_ERR_ARG;
        }
    } else {
        switch (epi) {
            case Q4EPI_F32: e = launch_nsb<Q4PRO_RMSNORM, Q4EPI_F32>(nsb, geo.ks, upw, grid, a, s); break;
            case Q4EPI_SWIGLU: e = launch_nsb<Q4PRO_RMSNORM, Q4EPI_SWIGLU>(nsb, geo.ks, upw, grid, a, s); break;
            case Q4EPI_ARGMAX: e = launch_nsb<Q4PRO_RMSNORM, Q4EPI_ARGMAX>(nsb, geo.ks, upw, grid, a, s); break;
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

namespace t2h {
// The plain and residual GEMV is built for K and N: a supported superblock
// count and N a multiple of the rows one unit covers.
bool q4k_matvec_shape_built(uint32_t k, uint32_t n) {
    if (validate_q4(k) != T2H_OK || n == 0) return false;
    return n % q4_geometry(k / 256, Q4EPI_F32).rpw == 0;
}
}  // namespace t2h

extern "C" int t2h_q4k_matvec(const void* x, const void* w, void* y, int out_dtype, const float* residual,
                              uint32_t m, uint32_t k, uint32_t n, void* stream) {
    if (!x || !w || !y) return T2H_ERR_NULL;
    int st = validate_q4(k);
    if (st) return st;
    if (m == 0 || n == 0) return T2H_OK;
    const uint32_t nsb = k / 256;
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
    const uint32_t rpw = q4_geometry(nsb, epi).rpw;
    if (n % rpw != 0) return T2H_ERR_SHAPE;
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
        st = q4k_launch(Q4PRO_BF16, epi, a, nsb, g_max_blocks, 0, s);
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
    const int pro = norm_w ? Q4PRO_RMSNORM : Q4PRO_BF16;
    int epi;
    if (out_dtype == T2H_DTYPE_F32) {
        epi = Q4EPI_F32;
    } else if (out_dtype == T2H_DTYPE_BF16 && !norm_w) {
        epi = Q4EPI_BF16;
    } else {
        return T2H_ERR_DTYPE;
    }
    const uint32_t rpw = q4_geometry(nsb, epi).rpw;
    Q4GemvArgs a = {};
    uint32_t total = 0;
    st = fill_parts(a, n_parts, w, y, n, rpw, &total);
    if (st) return st;
    a.x = x;
    a.norm_w = norm_w;
    a.eps = eps;
    a.n_units = total / rpw;
    return q4k_launch(pro, epi, a, nsb, norm_w ? g_max_blocks_norm : g_max_blocks, 0,
                      reinterpret_cast<hipStream_t>(stream));
}

extern "C" int t2h_q4k_rmsnorm_swiglu_matvec(const float* h, const float* norm_w, float eps, const void* w_gate,
                                             const void* w_up, void* act_out, uint32_t k, uint32_t n,
                                             void* stream) {
    if (!h || !norm_w || !w_gate || !w_up || !act_out) return T2H_ERR_NULL;
    int st = validate_q4(k);
    if (st) return st;
    const uint32_t nsb = k / 256;
    const uint32_t rpw = q4_geometry(nsb, Q4EPI_SWIGLU).rpw;
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
    return q4k_launch(Q4PRO_RMSNORM, Q4EPI_SWIGLU, a, nsb, g_max_blocks_norm, 0,
                      reinterpret_cast<hipStream_t>(stream));
}

extern "C" int t2h_q4k_lm_head_argmax_partial(const void* x, const float* norm_w, float eps, const void* w,
                                              uint32_t k, uint32_t n, float* partial_scores,
                                              uint32_t* partial_tokens, uint32_t num_partials, void* stream) {
    if (!x || !w || !partial_scores || !partial_tokens) return T2H_ERR_NULL;
    int st = validate_q4(k);
    if (st) return st;
    const uint32_t nsb = k / 256;
    const uint32_t rpw = q4_geometry(nsb, Q4EPI_ARGMAX).rpw;
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
    return q4k_launch(norm_w ? Q4PRO_RMSNORM : Q4PRO_BF16, Q4EPI_ARGMAX, a, nsb, 0, num_partials,
                      reinterpret_cast<hipStream_t>(stream));
}

// ----------------------------------------------- LM head of several sequences --
//
// The LM head + per-block argmax of up to Q4_HEAD_SEQS sequences that decode
// together (one step of a decoder group): the head's rows are streamed once and
// dotted with every sequence's normed x, each sequence keeping its own argmax.
// Per sequence the result is bit-identical to t2h_q4k_lm_head_argmax_partial
// with the RMSNorm prologue: the same x staging (block of 8 waves, the same
// sum-of-squares order), the same lane dots, the same units per block, and row
// sums over the 64 / RPW lanes that hold a row, which is what wave_sum gives for
// the single-sequence kernel's per-row masked sums (every other lane adds an
// exact zero).
namespace t2h {

constexpr int Q4_HEAD_SEQS = 4;

struct Q4HeadSeqsArgs {
    const float* h[Q4_HEAD_SEQS];  // fp32 residual streams [K]
    const float* norm_w;           // fp32 [K], the final RMSNorm weight
    const uint8_t* w;              // Q4_K rows [N, K]
    float* scores[Q4_HEAD_SEQS];   // [gridDim.x] each
    uint32_t* tokens[Q4_HEAD_SEQS];
    uint32_t n_units;
    uint32_t units_per_wave;
    uint32_t n_partials;  // slots per sequence; those past the grid get the empty pair
    float eps;
};

// Sum over the 16 lanes of a DPP row (every lane of the row gets it), in
// wave_sum's order.
__device__ __forceinline__ float row16_sum(float v) {
    v += dpp_f32<0xB1>(v);
    v += dpp_f32<0x4E>(v);
    v += dpp_f32<0x141>(v);
    v += dpp_f32<0x140>(v);
    return v;
}

template <int NSB, int NX>
__global__ __launch_bounds__(512) void q4k_lm_head_seqs_kernel(const Q4HeadSeqsArgs a) {
    constexpr int K = NSB * 256;
    constexpr int WPB = 8;
    constexpr int NT = WPB * 64;
    constexpr int RPW = 16 / cgcd(NSB, 16);
    constexpr int ROW_BYTES = NSB * 144;
    constexpr int NSTAGE = 4;
    static_assert(NSB == 4 || NSB == 16, "rows of 4 or 16 superblocks: one 16-superblock step per unit");
    static_assert(NX >= 1 && NX <= Q4_HEAD_SEQS, "1..4 sequences");

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int sbo = lane >> 2;
    const int g = lane & 3;
    const int rloc = sbo / NSB;  // row of the unit this lane's superblock belongs to (lanes 64/RPW per row)
    const int sbi = sbo % NSB;

    struct Stage {
        uint4 hdr, q0, q1;
    };
    auto issue = [&](uint32_t unit, Stage& st) {
        const uint8_t* base = a.w + (size_t)(unit * RPW + (uint32_t)rloc) * ROW_BYTES + (size_t)sbi * 144;
        st.hdr = load_u4(base);
        st.q0 = load_u4(base + 16 + g * 32);
        st.q1 = load_u4(base + 32 + g * 32);
    };
    const uint32_t wrow = blockIdx.x * WPB + wave;
    const uint32_t total_wrows = gridDim.x * WPB;
    const uint32_t last_unit = a.n_units - 1;
    auto clamp_unit = [&](uint32_t u) { return u < a.n_units ? u : last_unit; };
    const uint32_t n_iter = a.units_per_wave;
    Stage st[NSTAGE];

    // x of every sequence: RMSNorm (bf16-rounded) staged in LDS as fp16 pair words
    __shared__ __align__(16) uint32_t xp[NX][xp_words(K)];
    __shared__ float xsum[NX][K / 32];
    __shared__ float red[NX][WPB];
    constexpr int PT = (K + 4 * NT - 1) / (4 * NT);
    float4 hv[NX][PT], wv[PT];
#pragma unroll
    for (int j = 0; j < PT; ++j) {
        const int k = (j * NT + (int)threadIdx.x) * 4;
        const bool in = K % (4 * NT) == 0 || k < K;
        wv[j] = in ? *reinterpret_cast<const float4*>(a.norm_w + k) : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int x = 0; x < NX; ++x)
            hv[x][j] = in ? *reinterpret_cast<const float4*>(a.h[x] + k) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    issue(clamp_unit(wrow), st[0]);
#pragma unroll
    for (int x = 0; x < NX; ++x) {
        float ss = 0.0f;
#pragma unroll
        for (int j = 0; j < PT; ++j) {
            ss = fmaf(hv[x][j].x, hv[x][j].x, ss);
            ss = fmaf(hv[x][j].y, hv[x][j].y, ss);
            ss = fmaf(hv[x][j].z, hv[x][j].z, ss);
            ss = fmaf(hv[x][j].w, hv[x][j].w, ss);
        }
        ss = wave_sum(ss);
        if (lane == 0) red[x][wave] = ss;
    }
    __syncthreads();
#pragma unroll
    for (int x = 0; x < NX; ++x) {
        float total = 0.0f;
#pragma unroll
        for (int i = 0; i < WPB; ++i) total += red[x][i];
        const float inv = 1.0f / sqrtf(total / (float)K + a.eps);
#pragma unroll
        for (int j = 0; j < PT; ++j) {
            const int k = (j * NT + (int)threadIdx.x) * 4;
            if (K % (4 * NT) == 0 || k < K)
                stage_x4(xp[x], xsum[x], k, bf16_round(hv[x][j].x * inv * wv[j].x),
                         bf16_round(hv[x][j].y * inv * wv[j].y), bf16_round(hv[x][j].z * inv * wv[j].z),
                         bf16_round(hv[x][j].w * inv * wv[j].w));
        }
    }
    __syncthreads();
#pragma unroll
    for (int s = 1; s < NSTAGE; ++s)
        if ((uint32_t)s < n_iter) issue(clamp_unit(wrow + s * total_wrows), st[s]);
    XSlice16 xs[NX];
#pragma unroll
    for (int x = 0; x < NX; ++x) load_xslice16(xp[x], xsum[x], sbi, g, xs[x]);
    const Q4LaneConsts lc = q4k_lane_consts(g);

    // each lane keeps the best (score, token) of the rows its 64 / RPW-lane group covers
    float best_score[NX];
    uint32_t best_token[NX];
#pragma unroll
    for (int x = 0; x < NX; ++x) {
        best_score[x] = -3.4028234663852886e38f;
        best_token[x] = 0xffffffffu;
    }
    auto consume = [&](uint32_t u, const Stage& s) {
        const uint32_t row = u * RPW + (uint32_t)rloc;
#pragma unroll
        for (int x = 0; x < NX; ++x) {
            const float c = q4k_lane_dot(s.hdr, s.q0, s.q1, xs[x], lc);
            const float r = RPW == 4 ? row16_sum(c) : wave_sum(c);
            if (u < a.n_units && better_pair(r, row, best_score[x], best_token[x])) {
                best_score[x] = r;
                best_token[x] = row;
            }
        }
    };
    for (uint32_t i = 0; i < n_iter; i += NSTAGE) {
#pragma unroll
        for (int s = 0; s < NSTAGE; ++s) {
            const uint32_t ui = i + s;
            if (ui >= n_iter) break;  // wave-uniform
            consume(wrow + ui * total_wrows, st[s]);
            if (ui + NSTAGE < n_iter) issue(clamp_unit(wrow + (ui + NSTAGE) * total_wrows), st[s]);
        }
    }

    __shared__ float bs[NX][WPB];
    __shared__ uint32_t bt[NX][WPB];
#pragma unroll
    for (int x = 0; x < NX; ++x) {
        float sc = best_score[x];
        uint32_t tk = best_token[x];
        wave_argmax(sc, tk);
        if (lane == 0) {
            bs[x][wave] = sc;
            bt[x][wave] = tk;
        }
    }
    __syncthreads();
    if (threadIdx.x < (unsigned)NX) {
        const int x = threadIdx.x;
        float sc = bs[x][0];
        uint32_t tk = bt[x][0];
        for (int i = 1; i < WPB; ++i) {
            if (better_pair(bs[x][i], bt[x][i], sc, tk)) {
                sc = bs[x][i];
                tk = bt[x][i];
            }
        }
        a.scores[x][blockIdx.x] = sc;
        a.tokens[x][blockIdx.x] = tk;
        for (uint32_t slot = gridDim.x + blockIdx.x; slot < a.n_partials; slot += gridDim.x) {
            a.scores[x][slot] = -3.4028234663852886e38f;  // no row: loses to every row's (score, token)
            a.tokens[x][slot] = 0xffffffffu;
        }
    }
}

template <int NSB>
static hipError_t launch_head_seqs(uint32_t nx, dim3 grid, const Q4HeadSeqsArgs& a, hipStream_t s) {
    switch (nx) {
        case 1: hipLaunchKernelGGL((q4k_lm_head_seqs_kernel<NSB, 1>), grid, dim3(512), 0, s, a); break;
        case 2: hipLaunchKernelGGL((q4k_lm_head_seqs_kernel<NSB, 2>), grid, dim3(512), 0, s, a); break;
        case 3: hipLaunchKernelGGL((q4k_lm_head_seqs_kernel<NSB, 3>), grid, dim3(512), 0, s, a); break;
        case 4: hipLaunchKernelGGL((q4k_lm_head_seqs_kernel<NSB, 4>), grid, dim3(512), 0, s, a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace t2h

extern "C" int t2h_q4k_lm_head_argmax_partial_seqs(uint32_t n_seq, const float* const* h, const float* norm_w,
                                                   float eps, const void* w, uint32_t k, uint32_t n,
                                                   float* const* partial_scores, uint32_t* const* partial_tokens,
                                                   uint32_t num_partials, void* stream) {
    if (!h || !norm_w || !w || !partial_scores || !partial_tokens) return T2H_ERR_NULL;
    if (n_seq == 0 || n_seq > (uint32_t)Q4_HEAD_SEQS) return T2H_ERR_ARG;
    if (k != 1024 && k != 4096) return T2H_ERR_UNSUPPORTED;
    const uint32_t nsb = k / 256;
    const Q4Geometry geo = q4_geometry(nsb, Q4EPI_ARGMAX);
    if (n == 0 || n % geo.rpw) return T2H_ERR_SHAPE;
    if (num_partials == 0) return T2H_ERR_ARG;
    if (reinterpret_cast<uintptr_t>(norm_w) % 16) return T2H_ERR_ALIGN;
    if (reinterpret_cast<uintptr_t>(w) % 16) return T2H_ERR_ALIGN;  // 16-B superblock loads
    Q4HeadSeqsArgs a = {};
    for (uint32_t i = 0; i < n_seq; ++i) {
        if (!h[i] || !partial_scores[i] || !partial_tokens[i]) return T2H_ERR_NULL;
        if (reinterpret_cast<uintptr_t>(h[i]) % 16) return T2H_ERR_ALIGN;  // float4 loads
        a.h[i] = h[i];
        a.scores[i] = partial_scores[i];
        a.tokens[i] = partial_tokens[i];
    }
    a.norm_w = norm_w;
    a.w = static_cast<const uint8_t*>(w);
    a.eps = eps;
    a.n_units = n / geo.rpw;
    a.n_partials = num_partials;
    // One sequence: the single-sequence launch's geometry (num_partials blocks of 8 waves, its partials
    // bit for bit).  Several: above 128 VGPRs a CU holds one block of 8 waves, so the grid is one block per
    // CU (a second round of blocks would wait for the first); the unused slots get the empty pair, and the
    // selected (score, token) is the same, the order of better_pair being total.
    uint32_t blocks = num_partials;
    if (n_seq > 1) {
        int dev = 0, cus = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
            return T2H_ERR_HIP_BASE + (int)hipErrorInvalidDevice;
        blocks = num_partials < (uint32_t)cus ? num_partials : (uint32_t)cus;
    }
    a.units_per_wave = units_per_wave_for(a.n_units, blocks, geo);
    if (blocks_for(a.n_units, a.units_per_wave, geo) > blocks) return T2H_ERR_ARG;
    const dim3 grid(blocks);
    const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const hipError_t e = nsb == 4 ? launch_head_seqs<4>(n_seq, grid, a, s) : launch_head_seqs<16>(n_seq, grid, a, s);
    return e == hipSuccess ? T2H_OK : T2H_ERR_HIP_BASE + (int)e;
}
