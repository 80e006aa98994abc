// Persistent decode kernel: every transformer layer of one Qwen3 decode token
// in one launch (uniform Q4_K weights, bf16 KV cache, batch 1).
//
// Replaces the per-layer dispatch sequence of the reference's decode step,
// run_decode_layer(rt, layer_idx, cache_position=...) for every layer
// (src/models/optimized_qwen3/dispatch/decode_layer.py:60-136, driven from
// src/models/optimized_qwen3/run.py:142-172):
//   RMS_NORM_MUL + LINEAR_NOBIAS_Q4_K_QKV_MATVEC      -> phase QKV
//   RMS_NORM_ROPE_TRANSPOSE x2 + SDPA_DECODE_CACHE_WRITE -> phases ATTN, MERGE
//   LINEAR_NOBIAS_Q4_K_MATVEC_ADD (o_proj)            -> phase O
//   RMS_NORM_MUL + LINEAR_NOBIAS_Q4_K_QK_MATVEC + SWIGLU -> phase GATE_UP
//   LINEAR_NOBIAS_Q4_K_MATVEC_ADD (down_proj)         -> phase DOWN
// with the same arithmetic as the one-kernel-per-op path (csrc/gemv_q4k.hip,
// csrc/attn_decode.hip), so both produce the same hidden state.
//
// Why one launch.  On MI355X a dependent kernel in a HIP graph costs ~1.75 us
// before its first wave runs, and each GEMV then ramps up and drains on its
// own.  Here 256 resident blocks of 8 waves (one per CU) walk the phases and
// meet at a grid barrier between them: per-XCD-group counters feeding one
// global counter and a generation word, ~1.85 us, all with agent-scope
// relaxed atomics and bounded spins (a timed-out spin sets the status word
// and the block moves on, so the launch always ends).  Before each barrier a
// wave issues the weight loads of its share of the next phase, which do not
// depend on the barrier, so HBM keeps streaming while the grid waits.
//
// Coherence.  Activations that cross blocks (h, q|k|v, attention partials,
// attention output, SwiGLU output) are written and read with agent-scope
// atomic accesses (sc1): each XCD has its own L2, and plain accesses could hit
// a stale line.  A block's stores are complete (s_waitcnt) before it arrives
// at a barrier.  Weights and the KV cache rows read here are not written in
// the same launch, so they use ordinary loads.
#include "q4k_device.h"

namespace t2h {

constexpr int DL_BLOCKS = 256;
constexpr int DL_WAVES = 8;                    // waves per block
constexpr int DL_THREADS = DL_WAVES * 64;
constexpr int DL_NW = DL_BLOCKS * DL_WAVES;    // waves in the grid
constexpr int DL_D = 128;                      // head dim
constexpr int DL_ATT_POS = 32;                 // positions per wave per attention pass (two rows per lane)
constexpr int DL_ATT_SLOTS = DL_BLOCKS / 8;    // attention blocks per kv head (8 kv heads)
constexpr int DL_GROUPS = 8;                   // barrier groups
constexpr uint32_t DL_SPIN_LIMIT = 1u << 14;   // polls before a barrier gives up (~16 ms)

// Per-layer pointer table (device memory, DL_LAYER_PTRS uint64 per layer).
// DL_WQ points at the q, k and v rows stacked contiguously (6144 rows); DL_WK and
// DL_WV must point inside it at rows 4096 and 5120 (checked by the host).
enum DlLayerPtr {
    DL_WQ = 0, DL_WK, DL_WV, DL_WO, DL_WGATE, DL_WUP, DL_WDOWN,
    DL_IN_NORM, DL_POST_NORM, DL_Q_NORM, DL_K_NORM, DL_K_CACHE, DL_V_CACHE,
    DL_LAYER_PTRS
};

struct DlArgs {
    const uint64_t* layers;   // [n_layers][DL_LAYER_PTRS]
    uint32_t n_layers;
    float* h;                 // fp32 [HID] residual stream (in/out)
    const int32_t* pos_ptr;
    uint32_t s_cap;
    float eps;
    float theta;
    float* qkv;               // fp32 [QD + 2 KVD]
    float* attn;              // fp32 [QD]
    float* act;               // fp32 [MLP]
    float* part;              // attention partials [NK][SLOTS][GROUP][2 + D]
    uint32_t* bar;            // barrier words (zero before first use, monotonic after)
    uint32_t* status;         // set non-zero when a barrier spin timed out
};

// ------------------------------------------------------ coherent access ----

__device__ __forceinline__ float ld_coh(const float* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float2 ld_coh2(const float* p) {
    const uint64_t v = __hip_atomic_load(reinterpret_cast<const uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return make_float2(__uint_as_float((uint32_t)v), __uint_as_float((uint32_t)(v >> 32)));
}
__device__ __forceinline__ void st_coh(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_coh2(float* p, float a, float b) {
    const uint64_t v = (uint64_t)__float_as_uint(a) | ((uint64_t)__float_as_uint(b) << 32);
    __hip_atomic_store(reinterpret_cast<uint64_t*>(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ------------------------------------------------------------- barrier ----

struct DlBarrier {
    uint32_t* group;  // [DL_GROUPS] counters, 256 B apart
    uint32_t* all;    // group-complete counter
    uint32_t* gen;    // generation released
    uint32_t* status;
    uint32_t base;    // generation at launch
    uint32_t round;
};

__device__ __forceinline__ void dl_grid_barrier(DlBarrier& b) {
    ++b.round;
    // Every wave waits for its own stores to complete before the block
    // arrives.  The shared vectors are written with agent-scope (sc1) stores,
    // which complete once they are performed at the device coherence point, so
    // a completed store is visible to every later sc1 load on any XCD; a
    // workgroup-scope fence would not wait for them on this part.  The wait
    // also covers any load still in flight (vector memory counts retire in
    // order), so no weight load of the next phase is issued before a barrier.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0) {
        const uint32_t target = b.base + b.round;
        constexpr uint32_t per_group = DL_BLOCKS / DL_GROUPS;
        uint32_t* gc = b.group + 64 * (blockIdx.x % DL_GROUPS);
        const uint32_t prev = __hip_atomic_fetch_add(gc, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (prev + 1u == target * per_group) {
            const uint32_t g = __hip_atomic_fetch_add(b.all, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (g + 1u == target * DL_GROUPS)
                __hip_atomic_store(b.gen, target, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        uint32_t polls = 0;
        while ((int32_t)(__hip_atomic_load(b.gen, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) - target) < 0) {
            if (++polls > DL_SPIN_LIMIT) {
                __hip_atomic_store(b.status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
    }
    __syncthreads();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
}

struct DlAttnLds {
    float qs[4][4][36];                 // GROUP=4 q heads x 4 quarters x (32 dims + pad)
    float4 ps4[DL_WAVES][DL_ATT_POS];   // exp(score - m) per wave and position, one float per q head
    float wml[DL_WAVES][4][2];
    float2 wo[DL_WAVES][4][64];
    uint16_t knew[DL_D];
};

constexpr int DL_HSB = 16;   // hidden 4096 = 16 superblocks
constexpr int DL_MSB = 48;   // MLP 12288 = 48 superblocks
constexpr int DL_HID = DL_HSB * 256;
constexpr int DL_MLP = DL_MSB * 256;
constexpr int DL_QKV_ROWS = 32 * DL_D + 2 * 8 * DL_D;  // 6144

union DlShared {
    struct {
        uint32_t xp[DL_MLP / 2];
        float xsum[DL_MLP / 32];
        float red[DL_WAVES];
    } g;
    DlAttnLds at;
};

// ------------------------------------------------------------ GEMV phase ----

// Weights of one unit (one row of each of NG row groups), K = NSB*256: the
// header and the two 16-B nibble chunks of this lane's superblock per
// 16-superblock step.
template <int NSB, int NG>
struct DlUnit {
    static constexpr int NIT = NSB / 16;
    uint4 hdr[NG][NIT];
    uint4 q0[NG][NIT];
    uint4 q1[NG][NIT];
};

// Row pointers of a GEMV phase: NG == 2 reads row `row` of w0 and w1.
struct DlRows {
    const uint8_t* w0;  // rows of the matrix (QKV: q, k and v rows stacked in one allocation)
    const uint8_t* w1;  // NG == 2: the second matrix (up)
    uint32_t n_rows;
};

template <int NSB, int NG>
__device__ __forceinline__ void dl_issue_unit(DlUnit<NSB, NG>& u, const DlRows& r, uint32_t row) {
    constexpr int ROW_BYTES = NSB * 144;
    const int lane = threadIdx.x & 63;
    const int sbo = lane >> 2;
    const int g = lane & 3;
    row = row < r.n_rows ? row : r.n_rows - 1;
#pragma unroll
    for (int gi = 0; gi < NG; ++gi) {
        const uint8_t* base;
        base = (gi == 0 ? r.w0 : r.w1) + (size_t)row * ROW_BYTES;
#pragma unroll
        for (int it = 0; it < DlUnit<NSB, NG>::NIT; ++it) {
            const uint8_t* p = base + (size_t)(it * 16 + sbo) * 144;
            u.hdr[gi][it] = load_u4(p);
            u.q0[gi][it] = load_u4(p + 16 + g * 32);
            u.q1[gi][it] = load_u4(p + 32 + g * 32);
        }
    }
}

// Stage x (K values) in LDS as fp16 pair words + sub-block sums.  RMSNORM:
// x = bf16(h * rsqrt(mean(h^2) + eps) * w), h read coherently; otherwise x =
// bf16(src) with src an fp32 activation written by an earlier phase.
template <int K, bool RMSNORM>
__device__ __forceinline__ void dl_stage_x(uint32_t* xp, float* xsum, float* red, const float* src,
                                           const float* norm_w, float eps) {
    constexpr int PT = K / (4 * DL_THREADS);
    static_assert(K % (4 * DL_THREADS) == 0, "K must fill the block");
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    float4 hv[PT];
#pragma unroll
    for (int j = 0; j < PT; ++j) {
        const int k = (j * DL_THREADS + tid) * 4;
        const float2 a = ld_coh2(src + k);
        const float2 b = ld_coh2(src + k + 2);
        hv[j] = make_float4(a.x, a.y, b.x, b.y);
    }
    if constexpr (RMSNORM) {
        float4 wv[PT];
#pragma unroll
        for (int j = 0; j < PT; ++j) wv[j] = *reinterpret_cast<const float4*>(norm_w + (j * DL_THREADS + tid) * 4);
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
        for (int i = 0; i < DL_WAVES; ++i) total += red[i];
        const float inv = 1.0f / sqrtf(total / (float)K + eps);
#pragma unroll
        for (int j = 0; j < PT; ++j) {
            const int k = (j * DL_THREADS + tid) * 4;
            stage_x4(xp, xsum, k, bf16_round(hv[j].x * inv * wv[j].x), bf16_round(hv[j].y * inv * wv[j].y),
                     bf16_round(hv[j].z * inv * wv[j].z), bf16_round(hv[j].w * inv * wv[j].w));
        }
    } else {
#pragma unroll
        for (int j = 0; j < PT; ++j) {
            const int k = (j * DL_THREADS + tid) * 4;
            stage_x4(xp, xsum, k, bf16_round(hv[j].x), bf16_round(hv[j].y), bf16_round(hv[j].z),
                     bf16_round(hv[j].w));
        }
    }
    __syncthreads();
}

enum DlEpi { DL_EPI_STORE = 0, DL_EPI_RESID = 1, DL_EPI_SWIGLU = 2 };

// Wave-reduced dot products of one unit against the staged x, one x slice
// live at a time.
template <int NSB, int NG>
__device__ __forceinline__ void dl_dot_unit(const DlUnit<NSB, NG>& u, const uint32_t* xp, const float* xsum,
                                            const Q4LaneConsts& lc, float (&res)[NG]) {
    constexpr int NIT = DlUnit<NSB, NG>::NIT;
    const int lane = threadIdx.x & 63;
    const int sbo = lane >> 2;
    const int g = lane & 3;
    float acc[NG];
#pragma unroll
    for (int it = 0; it < NIT; ++it) {
        XSlice16 xs;
        load_xslice16(xp, xsum, it * 16 + sbo, g, xs);
#pragma unroll
        for (int gi = 0; gi < NG; ++gi) {
            const float c = q4k_lane_dot(u.hdr[gi][it], u.q0[gi][it], u.q1[gi][it], xs, lc);
            acc[gi] = it == 0 ? c : acc[gi] + c;
        }
    }
#pragma unroll
    for (int gi = 0; gi < NG; ++gi) res[gi] = wave_sum(acc[gi]);
}

//   STORE: y[row] = dot;  RESID: y[row] += dot;  SWIGLU: y[row] = bf16(silu(g) * u) (kept in fp32)
template <int NG, int EPI>
__device__ __forceinline__ void dl_store_row(float* y, uint32_t row, uint32_t n_rows, const float (&res)[NG]) {
    if ((threadIdx.x & 63) == 0 && row < n_rows) {
        if constexpr (EPI == DL_EPI_STORE) {
            st_coh(y + row, res[0]);
        } else if constexpr (EPI == DL_EPI_RESID) {
            st_coh(y + row, ld_coh(y + row) + res[0]);
        } else {
            st_coh(y + row, bf16_round(silu(res[0]) * res[NG - 1]));
        }
    }
}

// One GEMV phase over the wave's UPW units (rows wrow + i * DL_NW), streamed
// through a ring of R units.  The first R units are issued before x is
// staged, so the weight stream is in flight while the block normalises x;
// unit i + R is issued right after unit i has been reduced.  The loop is
// unrolled, so the ring is static registers, and the scheduling fences keep
// each refill after the reduction that frees its registers.
template <int NSB, int NG, int UPW, int R, int EPI, bool RMSNORM>
__device__ __forceinline__ void dl_gemv_phase(DlShared& sm, const DlRows& rows, uint32_t wrow, const float* x_src,
                                              const float* norm_w, float eps, float* y) {
    static_assert(R >= 1 && R <= UPW, "ring size");
    DlUnit<NSB, NG> u[UPW];
#pragma unroll
    for (int i = 0; i < R; ++i) dl_issue_unit(u[i], rows, wrow + (uint32_t)i * DL_NW);
    dl_stage_x<NSB * 256, RMSNORM>(sm.g.xp, sm.g.xsum, sm.g.red, x_src, norm_w, eps);
    const Q4LaneConsts lc = q4k_lane_consts(threadIdx.x & 3);
#pragma unroll
    for (int i = 0; i < UPW; ++i) {
        __builtin_amdgcn_sched_barrier(0);
        float res[NG];
        dl_dot_unit(u[i], sm.g.xp, sm.g.xsum, lc, res);
        dl_store_row<NG, EPI>(y, wrow + (uint32_t)i * DL_NW, rows.n_rows, res);
        __builtin_amdgcn_sched_barrier(0);
        if (i + R < UPW) dl_issue_unit(u[i + R], rows, wrow + (uint32_t)(i + R) * DL_NW);
    }
}

// --------------------------------------------------------- attention phase ----

// K and V rows of one wave's positions, loaded ahead of the scores.
struct DlAttnBank {
    uint4 kr[2][4];            // rows p_k and 16 + p_k: dims part*32 .. +31
    uint32_t vr[DL_ATT_POS];   // dims 2 lane, 2 lane + 1 of each position
};

__device__ __forceinline__ int dl_att_span(int L) {
    // positions per wave: the kv head's L positions over its DL_ATT_SLOTS * DL_WAVES waves
    return (L + DL_ATT_SLOTS * DL_WAVES - 1) / (DL_ATT_SLOTS * DL_WAVES);
}

__device__ __forceinline__ void dl_attn_issue(DlAttnBank& bk, const uint16_t* kc, const uint16_t* vc, int kvh, int p0,
                                              int L) {
    const int lane = threadIdx.x & 63;
    const int p_k = lane >> 2, part = lane & 3;
    const size_t stride = (size_t)8 * DL_D;
#pragma unroll
    for (int r = 0; r < 2; ++r) {
        const int p = min(p0 + 16 * r + p_k, L - 1);
        const uint16_t* krow = kc + (size_t)p * stride + (size_t)kvh * DL_D + part * 32;
#pragma unroll
        for (int i = 0; i < 4; ++i) bk.kr[r][i] = load_u4(krow + 8 * i);
    }
#pragma unroll
    for (int i = 0; i < DL_ATT_POS; ++i) {
        const int p = min(p0 + i, L - 1);
        bk.vr[i] = reinterpret_cast<const uint32_t*>(vc + (size_t)p * stride + (size_t)kvh * DL_D)[lane];
    }
}

__device__ __forceinline__ void dl_norm_rope(float x0, float x1, const float* w, bool has_w, float eps, float cs,
                                             float sn, bool rope, float& r0, float& r1) {
    const int lane = threadIdx.x & 63;
    float n0 = x0, n1 = x1;
    if (has_w) {
        const float ss = wave_sum(x0 * x0 + x1 * x1);
        const float inv = 1.0f / sqrtf(ss / (float)DL_D + eps);
        n0 = x0 * inv * w[lane];
        n1 = x1 * inv * w[lane + 64];
    }
    if (rope) {
        r0 = n0 * cs - n1 * sn;
        r1 = n1 * cs + n0 * sn;
    } else {
        r0 = n0;
        r1 = n1;
    }
}

// Block (kv head kvh, slot bs): wave w covers positions [p0, p0 + span) of the
// first L; the block's (max, sum, output) per q head goes to part[kvh][bs].
__device__ __forceinline__ void dl_attn_phase(const DlAttnBank& bk, DlAttnLds& sm, const DlArgs& a, const uint64_t* lp, int kvh,
                              int bs, int pos, int L) {
    constexpr int GROUP = 4;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int span = dl_att_span(L);
    const int p0 = (bs * DL_WAVES + wave) * span;
    int rows = L - p0;
    rows = rows < 0 ? 0 : (rows > span ? span : rows);
    const int S = (int)a.s_cap;
    const bool has_new = pos < S && pos >= p0 && pos < p0 + rows;
    const int rnew = pos - p0;
    const bool rope = a.theta > 0.0f;
    const float* q_norm = reinterpret_cast<const float*>(lp[DL_Q_NORM]);
    const float* k_norm = reinterpret_cast<const float*>(lp[DL_K_NORM]);
    uint16_t* kc = reinterpret_cast<uint16_t*>(lp[DL_K_CACHE]);
    uint16_t* vc = reinterpret_cast<uint16_t*>(lp[DL_V_CACHE]);
    const float* q = a.qkv;
    const float* kn = a.qkv + 32 * DL_D;
    const float* vn = a.qkv + 40 * DL_D;

    float cs = 1.0f, sn = 0.0f;
    if (rope && (wave < GROUP || has_new)) {
        const float inv_freq = exp2f(-(2.0f * (float)lane / (float)DL_D) * log2f(a.theta));
        sincosf((float)pos * inv_freq, &sn, &cs);
    }
    if (wave < GROUP) {
        const int hq = kvh * GROUP + wave;
        float r0, r1;
        dl_norm_rope(ld_coh(q + hq * DL_D + lane), ld_coh(q + hq * DL_D + lane + 64), q_norm, q_norm != nullptr,
                     a.eps, cs, sn, rope, r0, r1);
        const float scale = 1.0f / sqrtf((float)DL_D);
        sm.qs[wave][lane >> 5][lane & 31] = r0 * scale;
        sm.qs[wave][2 + (lane >> 5)][lane & 31] = r1 * scale;
    }
    uint32_t vnew = 0;
    if (has_new) {
        float k0, k1;
        dl_norm_rope(ld_coh(kn + kvh * DL_D + lane), ld_coh(kn + kvh * DL_D + lane + 64), k_norm, k_norm != nullptr,
                     a.eps, cs, sn, rope, k0, k1);
        const uint16_t kb0 = (uint16_t)f32_to_bf16_bits(k0), kb1 = (uint16_t)f32_to_bf16_bits(k1);
        sm.knew[lane] = kb0;
        sm.knew[lane + 64] = kb1;
        const float2 vv = ld_coh2(vn + kvh * DL_D + 2 * lane);
        vnew = pack_bf16x2(vv.x, vv.y);
        const size_t off = (size_t)pos * 8 * DL_D + (size_t)kvh * DL_D;
        kc[off + lane] = kb0;
        kc[off + lane + 64] = kb1;
        reinterpret_cast<uint32_t*>(vc + off)[lane] = vnew;
    }
    __syncthreads();

    const int p_k = lane >> 2, part = lane & 3;
    float mg[GROUP], lg[GROUP];
#pragma unroll
    for (int gg = 0; gg < GROUP; ++gg) {
        mg[gg] = -INFINITY;
        lg[gg] = 0.0f;
    }
    float s[2][GROUP];
    uint4 kr[2][4];
#pragma unroll
    for (int r = 0; r < 2; ++r) {
#pragma unroll
        for (int i = 0; i < 4; ++i) kr[r][i] = bk.kr[r][i];
        if (has_new && 16 * r + p_k == rnew) {
#pragma unroll
            for (int i = 0; i < 4; ++i) kr[r][i] = *reinterpret_cast<const uint4*>(&sm.knew[part * 32 + 8 * i]);
        }
#pragma unroll
        for (int gg = 0; gg < GROUP; ++gg) s[r][gg] = 0.0f;
    }
    // each q fragment read from LDS once and used for both K rows
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        float kf[2][8];
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            const uint4 kk = kr[r][i];
            kf[r][0] = bf16_bits_to_f32(kk.x & 0xffffu); kf[r][1] = bf16_bits_to_f32(kk.x >> 16);
            kf[r][2] = bf16_bits_to_f32(kk.y & 0xffffu); kf[r][3] = bf16_bits_to_f32(kk.y >> 16);
            kf[r][4] = bf16_bits_to_f32(kk.z & 0xffffu); kf[r][5] = bf16_bits_to_f32(kk.z >> 16);
            kf[r][6] = bf16_bits_to_f32(kk.w & 0xffffu); kf[r][7] = bf16_bits_to_f32(kk.w >> 16);
        }
#pragma unroll
        for (int gg = 0; gg < GROUP; ++gg) {
            const float4 qa = *reinterpret_cast<const float4*>(&sm.qs[gg][part][8 * i]);
            const float4 qb = *reinterpret_cast<const float4*>(&sm.qs[gg][part][8 * i + 4]);
#pragma unroll
            for (int r = 0; r < 2; ++r) {
                float t = s[r][gg];
                t = fmaf(qa.x, kf[r][0], t); t = fmaf(qa.y, kf[r][1], t);
                t = fmaf(qa.z, kf[r][2], t); t = fmaf(qa.w, kf[r][3], t);
                t = fmaf(qb.x, kf[r][4], t); t = fmaf(qb.y, kf[r][5], t);
                t = fmaf(qb.z, kf[r][6], t); t = fmaf(qb.w, kf[r][7], t);
                s[r][gg] = t;
            }
        }
    }
#pragma unroll
    for (int r = 0; r < 2; ++r) {
#pragma unroll
        for (int gg = 0; gg < GROUP; ++gg) {
            s[r][gg] += dpp_f32<0xB1>(s[r][gg]);
            s[r][gg] += dpp_f32<0x4E>(s[r][gg]);
        }
    }
    // softmax statistics over this wave's rows (both halves)
#pragma unroll
    for (int gg = 0; gg < GROUP; ++gg) {
        const bool v0 = p_k < rows, v1 = 16 + p_k < rows;
        const float a0 = v0 ? s[0][gg] : -INFINITY, a1 = v1 ? s[1][gg] : -INFINITY;
        const float m = wave_max(fmaxf(a0, a1));
        const float e0 = v0 ? expf(a0 - m) : 0.0f, e1 = v1 ? expf(a1 - m) : 0.0f;
        mg[gg] = m;
        lg[gg] = wave_sum(part == 0 ? e0 + e1 : 0.0f);
        if (part == 0) {
            reinterpret_cast<float*>(&sm.ps4[wave][p_k])[gg] = e0;
            reinterpret_cast<float*>(&sm.ps4[wave][16 + p_k])[gg] = e1;
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    float o0[GROUP], o1[GROUP];
#pragma unroll
    for (int gg = 0; gg < GROUP; ++gg) o0[gg] = o1[gg] = 0.0f;
    // P.V over the wave's positions (p >= rows carry p = 0).  Fully unrolled so
    // the V registers are indexed statically; the scheduling fence every 8
    // positions keeps the P reads from all being hoisted at once.
#pragma unroll
    for (int p = 0; p < DL_ATT_POS; ++p) {
        if (p % 8 == 0) __builtin_amdgcn_sched_barrier(0);
        const uint32_t vv = (has_new && p == rnew) ? vnew : bk.vr[p];
        const float v0 = bf16_bits_to_f32(vv & 0xffffu), v1 = bf16_bits_to_f32(vv >> 16);
        const float4 pr = sm.ps4[wave][p];
        o0[0] = fmaf(pr.x, v0, o0[0]); o1[0] = fmaf(pr.x, v1, o1[0]);
        o0[1] = fmaf(pr.y, v0, o0[1]); o1[1] = fmaf(pr.y, v1, o1[1]);
        o0[2] = fmaf(pr.z, v0, o0[2]); o1[2] = fmaf(pr.z, v1, o1[2]);
        o0[3] = fmaf(pr.w, v0, o0[3]); o1[3] = fmaf(pr.w, v1, o1[3]);
    }
#pragma unroll
    for (int gg = 0; gg < GROUP; ++gg) {
        sm.wo[wave][gg][lane] = make_float2(o0[gg], o1[gg]);
        if (lane == 0) {
            sm.wml[wave][gg][0] = mg[gg];
            sm.wml[wave][gg][1] = lg[gg];
        }
    }
    __syncthreads();
    // block partial: [kvh][bs][g] = (M, l, o[128])
    float* pb = a.part + (((size_t)kvh * DL_ATT_SLOTS + bs) * GROUP) * (2 + DL_D);
    for (int idx = tid; idx < GROUP * 64; idx += DL_THREADS) {
        const int gg = idx >> 6, dl = idx & 63;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < DL_WAVES; ++w) M = fmaxf(M, sm.wml[w][gg][0]);
        float l = 0.0f, r0 = 0.0f, r1 = 0.0f;
#pragma unroll
        for (int w = 0; w < DL_WAVES; ++w) {
            const float m = sm.wml[w][gg][0];
            const float f = m == -INFINITY ? 0.0f : expf(m - M);
            l = fmaf(f, sm.wml[w][gg][1], l);
            const float2 ov = sm.wo[w][gg][dl];
            r0 = fmaf(f, ov.x, r0);
            r1 = fmaf(f, ov.y, r1);
        }
        float* pg = pb + gg * (2 + DL_D);
        st_coh2(pg + 2 + 2 * dl, r0, r1);
        if (dl == 0) st_coh2(pg, M, l);
    }
}

// Head hq = blockIdx.x (< 32): merge the DL_ATT_SLOTS block partials of its kv head.
__device__ __forceinline__ void dl_merge_phase(DlAttnLds& sm, const DlArgs& a, int hq) {
    constexpr int GROUP = 4;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int kvh = hq / GROUP, gg = hq % GROUP;
    constexpr int PER_WAVE = DL_ATT_SLOTS / DL_WAVES;  // 4 partials per wave
    float2 ml[PER_WAVE], ov[PER_WAVE];
#pragma unroll
    for (int i = 0; i < PER_WAVE; ++i) {
        const int bs = wave * PER_WAVE + i;
        const float* pg = a.part + (((size_t)kvh * DL_ATT_SLOTS + bs) * GROUP + gg) * (2 + DL_D);
        ml[i] = ld_coh2(pg);
        ov[i] = ld_coh2(pg + 2 + 2 * lane);
    }
    float M = -INFINITY;
#pragma unroll
    for (int i = 0; i < PER_WAVE; ++i) M = fmaxf(M, ml[i].x);
    float l = 0.0f, r0 = 0.0f, r1 = 0.0f;
#pragma unroll
    for (int i = 0; i < PER_WAVE; ++i) {
        const float f = ml[i].x == -INFINITY ? 0.0f : expf(ml[i].x - M);
        l = fmaf(f, ml[i].y, l);
        r0 = fmaf(f, ov[i].x, r0);
        r1 = fmaf(f, ov[i].y, r1);
    }
    sm.wo[wave][0][lane] = make_float2(r0, r1);
    if (lane == 0) {
        sm.wml[wave][0][0] = M;
        sm.wml[wave][0][1] = l;
    }
    __syncthreads();
    if (wave == 0) {
        float Mt = -INFINITY;
#pragma unroll
        for (int w = 0; w < DL_WAVES; ++w) Mt = fmaxf(Mt, sm.wml[w][0][0]);
        float lt = 0.0f, a0 = 0.0f, a1 = 0.0f;
#pragma unroll
        for (int w = 0; w < DL_WAVES; ++w) {
            const float m = sm.wml[w][0][0];
            const float f = m == -INFINITY ? 0.0f : expf(m - Mt);
            lt = fmaf(f, sm.wml[w][0][1], lt);
            const float2 o = sm.wo[w][0][lane];
            a0 = fmaf(f, o.x, a0);
            a1 = fmaf(f, o.y, a1);
        }
        const float inv = 1.0f / lt;
        st_coh2(a.attn + hq * DL_D + 2 * lane, a0 * inv, a1 * inv);
    }
}

// ------------------------------------------------------------- the kernel ----

__global__ __launch_bounds__(DL_THREADS) void decode_layers_kernel(const DlArgs a) {
    __shared__ __align__(16) DlShared sm;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t wrow = blockIdx.x * DL_WAVES + wave;
    DlBarrier bar;
    bar.group = a.bar;
    bar.all = a.bar + 64 * DL_GROUPS;
    bar.gen = a.bar + 64 * (DL_GROUPS + 1);
    bar.status = a.status;
    bar.base = __hip_atomic_load(bar.gen, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    bar.round = 0;
    const int pos = *a.pos_ptr;
    const int L = pos + 1 < (int)a.s_cap ? pos + 1 : (int)a.s_cap;
    const int kvh = blockIdx.x % 8, bs = blockIdx.x / 8;

    typedef const __attribute__((address_space(4))) uint64_t* const_table_t;
    // the layer table is read-only for the launch: constant address space, scalar loads
    auto layer_ptr = [&](uint32_t layer, int field) -> uint64_t {
        const const_table_t tbl = (const_table_t)(a.layers + (size_t)layer * DL_LAYER_PTRS);
        return tbl[field];
    };
    auto qkv_rows = [&](uint32_t layer) {
        DlRows r;
        r.w0 = r.w1 = reinterpret_cast<const uint8_t*>(layer_ptr(layer, DL_WQ));  // q | k | v rows, contiguous
        r.n_rows = DL_QKV_ROWS;
        return r;
    };
    auto o_rows = [&](uint32_t layer) {
        DlRows r;
        r.w0 = r.w1 = reinterpret_cast<const uint8_t*>(layer_ptr(layer, DL_WO));
        r.n_rows = DL_HID;
        return r;
    };
    auto gu_rows = [&](uint32_t layer) {
        DlRows r;
        r.w0 = reinterpret_cast<const uint8_t*>(layer_ptr(layer, DL_WGATE));
        r.w1 = reinterpret_cast<const uint8_t*>(layer_ptr(layer, DL_WUP));
        r.n_rows = DL_MLP;
        return r;
    };
    auto down_rows = [&](uint32_t layer) {
        DlRows r;
        r.w0 = r.w1 = reinterpret_cast<const uint8_t*>(layer_ptr(layer, DL_WDOWN));
        r.n_rows = DL_HID;
        return r;
    };
    const int span = dl_att_span(L);
    const int att_p0 = (bs * DL_WAVES + wave) * span;

    for (uint32_t layer = 0; layer < a.n_layers; ++layer) {
        // ---- Q|K|V: RMSNorm(h) . [Wq; Wk; Wv]^T
        dl_gemv_phase<DL_HSB, 1, 3, 3, DL_EPI_STORE, true>(sm, qkv_rows(layer), wrow, a.h,
                                                          reinterpret_cast<const float*>(layer_ptr(layer, DL_IN_NORM)),
                                                          a.eps, a.qkv);
        dl_grid_barrier(bar);
        // ---- attention split
        {
            uint64_t lp[DL_LAYER_PTRS];
#pragma unroll
            for (int i = 0; i < DL_LAYER_PTRS; ++i) lp[i] = layer_ptr(layer, i);
            DlAttnBank bk;
            dl_attn_issue(bk, reinterpret_cast<const uint16_t*>(lp[DL_K_CACHE]),
                          reinterpret_cast<const uint16_t*>(lp[DL_V_CACHE]), kvh, att_p0, L);
            dl_attn_phase(bk, sm.at, a, lp, kvh, bs, pos, L);
        }
        dl_grid_barrier(bar);
        // ---- attention merge
        if (blockIdx.x < 32) dl_merge_phase(sm.at, a, blockIdx.x);
        dl_grid_barrier(bar);
        // ---- o_proj + residual
        dl_gemv_phase<DL_HSB, 1, 2, 2, DL_EPI_RESID, false>(sm, o_rows(layer), wrow, a.attn, nullptr, a.eps, a.h);
        dl_grid_barrier(bar);
        // ---- RMSNorm + gate|up + SwiGLU
        dl_gemv_phase<DL_HSB, 2, 6, 3, DL_EPI_SWIGLU, true>(sm, gu_rows(layer), wrow, a.h,
                                                           reinterpret_cast<const float*>(layer_ptr(layer, DL_POST_NORM)),
                                                           a.eps, a.act);
        dl_grid_barrier(bar);
        // ---- down + residual
        dl_gemv_phase<DL_MSB, 1, 2, 2, DL_EPI_RESID, false>(sm, down_rows(layer), wrow, a.act, nullptr, a.eps, a.h);
        if (layer + 1 < a.n_layers) dl_grid_barrier(bar);
    }
}

static size_t dl_align(size_t v) { return (v + 255) & ~(size_t)255; }

struct DlLayout {
    size_t qkv, attn, act, part, bar, total;
};

static DlLayout dl_layout() {
    DlLayout l;
    size_t off = 0;
    l.bar = off;
    off += dl_align(4 * 64 * (DL_GROUPS + 2) + 4);
    l.qkv = off;
    off += dl_align((size_t)DL_QKV_ROWS * 4);
    l.attn = off;
    off += dl_align((size_t)32 * DL_D * 4);
    l.act = off;
    off += dl_align((size_t)DL_MLP * 4);
    l.part = off;
    off += dl_align((size_t)8 * DL_ATT_SLOTS * 4 * (2 + DL_D) * 4);
    l.total = off;
    return l;
}

static int g_dl_fits = -1;  // cached residency check: 1 = 256 blocks fit at once

static bool dl_grid_fits() {
    if (g_dl_fits >= 0) return g_dl_fits == 1;
    int dev = 0, cus = 0, per_cu = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, decode_layers_kernel, DL_THREADS, 0) != hipSuccess) {
        g_dl_fits = 0;
        return false;
    }
    g_dl_fits = (cus * per_cu >= DL_BLOCKS) ? 1 : 0;
    return g_dl_fits == 1;
}

}  // namespace t2h

using namespace t2h;

extern "C" size_t t2h_qwen3_decode_layers_workspace_bytes(uint32_t hidden, uint32_t mlp, uint32_t nh, uint32_t nk,
                                                         uint32_t d) {
    if (hidden != DL_HID || mlp != DL_MLP || nh != 32 || nk != 8 || d != DL_D) return 0;
    return dl_layout().total;
}

extern "C" int t2h_qwen3_decode_layers(const uint64_t* layer_table, uint32_t n_layers, uint32_t hidden, uint32_t mlp,
                                       uint32_t nh, uint32_t nk, uint32_t d, uint32_t s_cap, float* h,
                                       const int32_t* cache_position, float eps, float theta, void* workspace,
                                       size_t workspace_bytes, uint32_t* status, void* stream) {
    if (!layer_table || !h || !cache_position || !workspace || !status) return T2H_ERR_NULL;
    if (hidden != DL_HID || mlp != DL_MLP || nh != 32 || nk != 8 || d != DL_D) return T2H_ERR_UNSUPPORTED;
    if (n_layers == 0) return T2H_OK;
    if (s_cap == 0) return T2H_ERR_SHAPE;
    if ((size_t)(s_cap + DL_ATT_SLOTS * DL_WAVES - 1) / (DL_ATT_SLOTS * DL_WAVES) > DL_ATT_POS)
        return T2H_ERR_UNSUPPORTED;  // more than 32 positions per wave
    const DlLayout l = dl_layout();
    if (workspace_bytes < l.total) return T2H_ERR_WORKSPACE;
    if (reinterpret_cast<uintptr_t>(workspace) % 256 != 0) return T2H_ERR_ALIGN;
    if (!dl_grid_fits()) return T2H_ERR_UNSUPPORTED;
    uint8_t* ws = reinterpret_cast<uint8_t*>(workspace);
    DlArgs a;
    a.layers = layer_table;
    a.n_layers = n_layers;
    a.h = h;
    a.pos_ptr = cache_position;
    a.s_cap = s_cap;
    a.eps = eps;
    a.theta = theta;
    a.qkv = reinterpret_cast<float*>(ws + l.qkv);
    a.attn = reinterpret_cast<float*>(ws + l.attn);
    a.act = reinterpret_cast<float*>(ws + l.act);
    a.part = reinterpret_cast<float*>(ws + l.part);
    a.bar = reinterpret_cast<uint32_t*>(ws + l.bar);
    a.status = status;
    hipLaunchKernelGGL(decode_layers_kernel, dim3(DL_BLOCKS), dim3(DL_THREADS), 0,
                       reinterpret_cast<hipStream_t>(stream), a);
    T2H_LAUNCH_CHECK();
    return T2H_OK;
}
