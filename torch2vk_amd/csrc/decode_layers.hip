// Persistent decode kernel: every transformer layer of one Qwen3 decode token
// in one launch (uniform Q4_K weights, bf16 KV cache, batch 1).  Built for the
// Qwen3-8B shape (hidden 4096, MLP 12288, 32/8 heads) and the Qwen3-0.6B shape
// (hidden 1024, MLP 3072, 16/8 heads); head_dim 128 and 8 kv heads in both.
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
// own.  Here 256 resident blocks of 8 waves (one per CU) walk the phases of
// every layer without a grid barrier: each phase first issues the weight (or
// KV-cache) loads of its share, which depend on nothing, and only then waits
// for its input vector, so HBM keeps streaming while the previous phase
// finishes elsewhere on the chip.
//
// Data flow instead of barriers.  Every element of a vector that crosses
// blocks (h, q|k|v, attention partials, attention output, SwiGLU output) is
// stored together with an epoch in one single-copy-atomic word: fp32 + u32
// epoch in 8 bytes, or bf16 + u16 epoch in 4 bytes.  A consumer loads the
// words it needs and re-loads until every epoch is the one this (launch,
// layer, phase) writes, so a producer never waits for its stores to complete
// and no block waits for the whole grid.  Epochs come from a launch counter
// in the workspace (advanced by block 0 at the end of every launch), so a
// value left from an earlier write never carries the expected epoch.  Spins
// are bounded: a consumer that gives up sets the status word and goes on, so
// the launch always ends (its results are then invalid).
//
// A buffer is rewritten only after every reader of its previous contents has
// finished: each phase reads the complete output of the phase before it, so a
// block that has the input of phase P + 1 knows that every block has passed
// phase P - 1.  Cross-block words are written and read with agent-scope atomic
// accesses (sc1): each XCD has its own L2, and plain accesses could hit a stale
// line.  Weights and the KV cache rows read here are not written in the same
// launch (except the new row, which its owner substitutes), so they use
// ordinary loads.
#include <atomic>
#include <mutex>
#include <type_traits>

#include "q4k_device.h"


namespace t2h {

constexpr int DL_BLOCKS = 256;
constexpr int DL_WAVES = 8;                    // waves per block
constexpr int DL_THREADS = DL_WAVES * 64;
constexpr int DL_NW = DL_BLOCKS * DL_WAVES;    // waves in the grid
constexpr int DL_D = 128;                      // head dim
constexpr int DL_ATT_POS = 32;                 // positions per wave per attention pass (two rows per lane)
constexpr int DL_ATT_SLOTS = DL_BLOCKS / 8;    // attention blocks per kv head (8 kv heads)
#ifndef DL_SPIN_LOG2
#define DL_SPIN_LOG2 14
#endif
constexpr uint32_t DL_SPIN_LIMIT = 1u << DL_SPIN_LOG2;
// weight units per wave issued before a GEMV phase's input is awaited
#ifndef DL_PRE_QKV
#define DL_PRE_QKV 1
#endif
#ifndef DL_PRE_O
#define DL_PRE_O 1
#endif
#ifndef DL_PRE_GU
#define DL_PRE_GU 1
#endif
#ifndef DL_PRE_DOWN
#define DL_PRE_DOWN 1
#endif   // polls before a consumer gives up (~16 ms)
// o_proj units issued once the attention phase has its q, so that they stream during the attention
// arithmetic and the merge (0: when the o_proj phase begins, like every other phase's units).
#ifndef DL_O_EARLY
#define DL_O_EARLY 2
#endif

struct DlNoHook {
    __device__ void operator()() const {}
};

// Per-layer table (device memory, DL_LAYER_PTRS uint64 per layer): the
// pointers, then the layer's weight types (DL_WTYPES bits).  DL_WQ points at
// the q and k rows stacked contiguously (q_dim + kv_dim rows), followed by the
// v rows when v is Q4_K too; DL_WK must point at row q_dim of it, and so must
// DL_WV at row q_dim + kv_dim when v is Q4_K (checked by the host).  A Q6_K v
// (DL_WT_V_Q6) or down (DL_WT_DOWN_Q6) is an allocation of its own: the
// Q4_K_M policy's more-bits layers.
enum DlLayerPtr {
    DL_WQ = 0, DL_WK, DL_WV, DL_WO, DL_WGATE, DL_WUP, DL_WDOWN,
    DL_IN_NORM, DL_POST_NORM, DL_Q_NORM, DL_K_NORM, DL_K_CACHE, DL_V_CACHE, DL_WTYPES,
    DL_LAYER_PTRS
};
enum DlWeightTypes : uint32_t { DL_WT_V_Q6 = 1u, DL_WT_DOWN_Q6 = 2u };
constexpr uint32_t DL_MAX_LAYERS = 64;  // layers per launch (the table is held in LDS)

struct DlArgs {
    const uint64_t* layers;   // [n_layers][DL_LAYER_PTRS]
    uint32_t n_layers;
    float* h;                 // fp32 [HID] residual stream (in/out, plain)
    const int32_t* pos_ptr;
    uint32_t s_cap;
    float eps;
    float theta;
    uint32_t* ctl;            // [0]: launches completed (epoch base)
    uint64_t* h_ll;           // [HID] fp32 + epoch: h after o_proj / down_proj
    uint64_t* qkv_ll;         // [QD + 2 KVD] fp32 + epoch
    uint64_t* part_ll;        // attention partials [NK][SLOTS][GROUP][2 + D], fp32 + epoch
    uint32_t* attn_ll;        // [QD] bf16 + epoch16: attention output
    uint32_t* act_ll;         // [MLP] bf16 + epoch16: SwiGLU output
    uint32_t* status;         // set non-zero when a consumer spin timed out
    uint64_t* trace;          // phase timestamps (the traced build only): [layer][phase][block][DL_TR_SLOTS]
};

// Phase timeline of the traced instantiation: per (layer, phase, block) the
// 100 MHz real-time clock at the phase's start, when its input is in hand,
// after its first unit is reduced (GEMV) or its softmax (attention), at its
// end, and the number of polls its first wave made for the input.
// Attention only: after the scores (DL_TR_A_SCORES), after P.V (DL_TR_A_PV) and after the waves' partials
// are merged in LDS (DL_TR_A_MERGED), each as seen by wave 0.
enum DlTraceSlot {
    DL_TR_BEGIN = 0, DL_TR_READY, DL_TR_FIRST, DL_TR_END, DL_TR_POLLS, DL_TR_A_SCORES, DL_TR_A_PV, DL_TR_A_MERGED,
    DL_TR_SLOTS = 8
};
constexpr int DL_TR_PHASES = 6;  // qkv, attention, merge, o, gate|up, down

__device__ __forceinline__ uint64_t* dl_trace_at(const DlArgs& a, uint32_t layer, int phase) {
    return a.trace == nullptr ? nullptr
                              : a.trace + (((size_t)layer * DL_TR_PHASES + phase) * DL_BLOCKS + blockIdx.x) * DL_TR_SLOTS;
}
__device__ __forceinline__ void dl_stamp(uint64_t* tr, int slot) {
    if (tr != nullptr && threadIdx.x == 0) tr[slot] = __builtin_amdgcn_s_memrealtime();
}

// The thread index as an opaque value: per-lane offsets derived from it are
// recomputed in every phase instead of being hoisted out of the layer loop,
// where they would stay live across the attention phase (the kernel's
// register peak) and be spilled.
__device__ __forceinline__ int dl_tid() {
    int t;
    asm volatile("v_mov_b32 %0, %1" : "=v"(t) : "v"((int)threadIdx.x));
    return t;
}

// A device address from the layer table as a global-address-space pointer:
// accesses through it compile to global_* instructions, which count only in
// vmcnt.  Through a generic pointer they would be FLAT instructions, which
// also count in lgkmcnt, so every LDS wait and every barrier would wait for
// all weight loads still in flight, and no prefetch could run past one.
template <class T>
__device__ __forceinline__ T* dl_gptr(uint64_t v) {
    return (T*)(__attribute__((address_space(1))) T*)v;
}

// ------------------------------------------------- epoch-tagged words ----

// Epoch ids of the vectors a layer writes.
enum DlEpoch { DL_E_QKV = 0, DL_E_PART, DL_E_ATTN, DL_E_H_O, DL_E_ACT, DL_E_H_DOWN, DL_E_PER_LAYER };

__device__ __forceinline__ uint32_t dl_epoch(uint32_t seq, uint32_t layer, int id) {
    return (seq + 1u) * 256u + layer * DL_E_PER_LAYER + (uint32_t)id;  // never 0 (zeroed workspace)
}

__device__ __forceinline__ uint64_t ll_load(const uint64_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void ll_store(uint64_t* p, uint64_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// fp32 value + 32-bit epoch
__device__ __forceinline__ void ll_put32(uint64_t* p, float v, uint32_t e) {
    ll_store(p, (uint64_t)__float_as_uint(v) | ((uint64_t)e << 32));
}
__device__ __forceinline__ float ll_val32(uint64_t w) { return __uint_as_float((uint32_t)w); }
__device__ __forceinline__ bool ll_ok32(uint64_t w, uint32_t e) { return (uint32_t)(w >> 32) == e; }
// two bf16 values, each with a 16-bit epoch, in one 8-byte word (element 2i in the low half)
__device__ __forceinline__ uint64_t ll_pack16x2(float a, float b, uint32_t e) {
    const uint64_t lo = f32_to_bf16_bits(a) | ((e & 0xffffu) << 16);
    const uint64_t hi = f32_to_bf16_bits(b) | ((e & 0xffffu) << 16);
    return lo | (hi << 32);
}
__device__ __forceinline__ bool ll_ok16x2(uint64_t w, uint32_t e) {
    const uint32_t e16 = e & 0xffffu;
    return ((uint32_t)(w >> 16) & 0xffffu) == e16 && (uint32_t)(w >> 48) == e16;
}
__device__ __forceinline__ void ll_put16(uint32_t* p, float v, uint32_t e) {
    __hip_atomic_store(p, f32_to_bf16_bits(v) | ((e & 0xffffu) << 16), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Where a wait gave up: status = DL_STATUS_TIMEOUT | layer << 8 | phase.
enum DlWaitSite { DL_W_QKV = 1, DL_W_ATTN_Q, DL_W_ATTN_KV, DL_W_MERGE, DL_W_O, DL_W_GU, DL_W_DOWN };
constexpr uint32_t DL_STATUS_TIMEOUT = 0x80000000u;

// Load N words (addr(i)) until ok(i, word) holds for all of them; bounded.
template <int N, class Addr, class Ok>
__device__ __forceinline__ uint32_t ll_wait(uint64_t (&w)[N], Addr addr, Ok ok, uint32_t* status, uint32_t site) {
    uint32_t polls = 0;
    for (;; ++polls) {
#pragma unroll
        for (int i = 0; i < N; ++i) w[i] = ll_load(addr(i));
        bool all = true;
#pragma unroll
        for (int i = 0; i < N; ++i) all = all && ok(i, w[i]);
        if (all) break;
        if (polls >= DL_SPIN_LIMIT) {
            __hip_atomic_store(status, DL_STATUS_TIMEOUT | site, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            break;
        }
        __builtin_amdgcn_s_sleep(1);
    }
    return polls;
}

typedef __bf16 dl_bf16x8_t __attribute__((ext_vector_type(8)));
typedef float dl_f32x4_t __attribute__((ext_vector_type(4)));

// V rows staged for the matrix-core P.V: [position][dims], padded to 272 B so that the transposing reads of
// 16 rows at one column spread over the banks
constexpr int DL_VROW = DL_D + 8;

template <int GROUP, bool PV_MFMA>
struct DlAttnLds {
    // each wave's V rows, read back transposed (ds_read_b64_tr_b16) as the B operand of P.V (matrix-core P.V)
    alignas(16) uint16_t vst[PV_MFMA ? DL_WAVES : 1][DL_ATT_POS * DL_VROW];
    // the block's q heads, normalised, rotated and scaled, as bf16 hi + lo parts (q = hi + lo to 2^-17)
    uint16_t qhi[GROUP][DL_D];
    uint16_t qlo[GROUP][DL_D];
    float wml[DL_WAVES][GROUP][2];
    // each wave's P.V: [dim][head] (heads 0 .. GROUP-1 of 4) from the matrix cores, or [head][dim pair] as
    // float2 from the VALU
    float4 wo[DL_WAVES][DL_D];
    float2 mo[DL_WAVES][64];               // the merge: each wave's combine of its partials
    uint16_t knew[DL_D];                   // the new position's K and V rows (bf16), for the wave holding it
    uint16_t vnew[DL_D];
};

constexpr int dl_max3(int a, int b, int c) { return a > b ? (a > c ? a : c) : (b > c ? b : c); }

// Model shape (8 kv heads of 128) and, per GEMV phase, the units per wave, the
// ring depth and the units issued before the input is awaited.
template <int HSB_, int MSB_, int NH_, int QKV_U, int QKV_R, int QKV_P, int O_U, int O_R, int O_P, int GU_U,
          int GU_R, int GU_P, int DN_U, int DN_R, int DN_P, bool PV_MFMA, int NB_ = DL_BLOCKS, bool O_LATE = false>
struct DlShape {
    // blocks per sequence: the launch's 256 blocks run 256 / NB sequences side by side
    static constexpr int NB = NB_, NSEQ = DL_BLOCKS / NB_, NW = NB_ * DL_WAVES, ATT_SLOTS = NB_ / 8;
    static_assert(NB == DL_BLOCKS || NB == 64, "one sequence, or four of 64 blocks");
    static constexpr int HSB = HSB_;             // hidden / 256 (superblocks)
    static constexpr int MSB = MSB_;             // MLP / 256
    static constexpr int NH = NH_;               // q heads
    static constexpr int NK = 8;                 // kv heads
    static constexpr int GROUP = NH / NK;
    static constexpr int QSB = NH * DL_D / 256;  // q_dim / 256: the o_proj row length
    static constexpr int HID = HSB * 256, MLP = MSB * 256, QD = NH * DL_D, KVD = NK * DL_D;
    static constexpr int QKV_ROWS = QD + 2 * KVD;
    static constexpr int KMAX = dl_max3(HID, MLP, QD);
    static constexpr int qkv_u = QKV_U, qkv_r = QKV_R, qkv_p = QKV_P, o_u = O_U, o_r = O_R, o_p = O_P;
    static constexpr int gu_u = GU_U, gu_r = GU_R, gu_p = GU_P, dn_u = DN_U, dn_r = DN_R, dn_p = DN_P;
    // attention P.V on the matrix cores (V transposed through LDS) or on the VALU (P broadcast by DPP):
    // measured faster for the 8B shape (4 q heads, 17 positions per wave at 4096) and slower for the 0.6B
    // one (2 q heads, 7 positions per wave at 1540)
    static constexpr bool pv_mfma = PV_MFMA;
    // the attention phase issues the early o_proj units after the scores instead of as soon as q is in hand:
    // measured 0.3-0.7 % faster per launch for the 8B shape at KV 4096 (alternating runs on one GPU), 0.8 %
    // slower for the 0.6B one
    static constexpr bool o_late = O_LATE;
    static_assert(NH % NK == 0 && NH / NK <= 4, "GQA group of 1..4 q heads");
};
#ifndef DL_QKV_SKIP
#define DL_QKV_SKIP 1
#endif
#ifndef DL_R_QKV
#define DL_R_QKV 2
#endif
#ifndef DL_R_O
#define DL_R_O 2
#endif
#ifndef DL_R_GU
#define DL_R_GU 2
#endif
#ifndef DL_R_DOWN
#define DL_R_DOWN 2
#endif
using DlQwen3_8B = DlShape<16, 48, 32, 3, DL_R_QKV, DL_PRE_QKV, 2, DL_R_O, DL_PRE_O, 6, DL_R_GU, DL_PRE_GU, 2, DL_R_DOWN,
                           DL_PRE_DOWN, true, DL_BLOCKS, true>;
using DlQwen3_0_6B = DlShape<4, 12, 16, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, false>;
// Qwen3-1.7B (hidden 2048, MLP 6144, 16 / 8 heads): rows of 8 and 24 superblocks, 2 rows a unit; Q|K|V one unit
// per wave, gate|up two, o and down spread.  The Q|K|V unit is issued once h is staged (647 against 654 us per
// launch at KV 4096, 551 against 555 at 192; down after its input, a ring of one gate|up unit, late o_proj
// units and matrix-core P.V measured equal or slower)
using DlQwen3_1_7B = DlShape<8, 24, 16, 1, 1, 0, 1, 1, 1, 2, 2, 1, 1, 1, 1, false>;
// four 0.6B sequences of 64 blocks each: every phase's units over 512 waves (Q|K|V 2 per wave, o 1, gate|up 2,
// down spread), attention over 8 blocks per kv head.  The down units are issued once the input is staged, not
// before the wait: 679 against 694 us per launch at KV 1540 (the single-sequence shapes measured slower so)
using DlQwen3_0_6B_x4 = DlShape<4, 12, 16, 2, 2, 1, 1, 1, 1, 2, 2, 1, 1, 1, 0, false, 64>;

constexpr int DL_HOLD = 4;  // residual rows a wave owns in one phase, at most

template <class S>
union DlShared {
    static constexpr int NB = S::NB;
    struct {
        uint32_t xp[xp_words(S::KMAX)];
        float xsum[S::KMAX / 32];
        float xsum16[S::KMAX / 16];  // sums of 16 values: the Q6_K units' scale groups
        float red[DL_WAVES];
        float hold[DL_WAVES * DL_HOLD];  // residual epilogue: the old h of the block's rows [wave][row]
    } g;
    DlAttnLds<S::GROUP, S::pv_mfma> at;
};

// ------------------------------------------------------------ GEMV phase ----

// Weights of one unit, K = NSB*256: RPW consecutive rows of each of NG row
// groups, streamed in NIT steps of 16 superblocks; per step a lane holds a
// quarter of superblock (step * 16 + lane / 4) of the unit (row = that / NSB).
// RPW = 1 for rows of 16, 32, 48 superblocks.
//   Q4_K: the header and the lane's two 16-B nibble chunks (hdr, q0, q1).
//   Q6_K: piece lane % 4 (half h = piece / 2, values l0 = 16 (piece % 2) ..
//         l0 + 15 of each of the half's 4 parts of 32): the 16-B ql chunks of
//         parts 0|2 and 1|3 (hdr, q0), the 16-B qh chunk (q1), the half's 8
//         int8 scales (sc) and d (d).
// The fields a format does not use are never touched, so they take no
// registers.
template <int NSB, int NG>
struct DlUnit {
    static constexpr int RPW = 16 / cgcd(NSB, 16);
    static constexpr int NIT = NSB * RPW / 16;
    uint4 hdr[NG][NIT];
    uint4 q0[NG][NIT];
    uint4 q1[NG][NIT];
    uint2 sc[NG][NIT];
    uint32_t d[NG][NIT];
};

// Unit formats of a GEMV phase: every unit Q4_K; Q4_K with the rows from
// DlRows::n_rows4 on in Q6_K (each wave's last unit slot may be one of those);
// every unit Q6_K.
enum DlFmt { DL_FMT_Q4 = 0, DL_FMT_Q4_TAIL6 = 1, DL_FMT_Q6 = 2 };

// Unit i of wave `wave` of this block, among the NB blocks of its sequence
// (blockIdx.x % NB: one sequence, or one of 256 / NB).  Block-major when every
// wave has a unit; SPREAD (fewer units than waves): across the blocks first, so
// that every CU streams a share.
// SPREAD with `skip`: the first `skip` blocks of the sequence take no unit (their index is past every unit) and
// the units spread over the others.
template <bool SPREAD, int NB>
__device__ __forceinline__ uint32_t dl_unit(uint32_t wave, uint32_t i, uint32_t skip = 0) {
    constexpr uint32_t NW = NB * DL_WAVES;
    const uint32_t lb = blockIdx.x % NB;
    if (SPREAD && skip != 0) return lb < skip ? 0xffffffffu : wave * (NB - skip) + (lb - skip) + i * NW;
    return SPREAD ? wave * NB + lb + i * NW : lb * DL_WAVES + wave + i * NW;
}

// Row pointers of a GEMV phase: NG == 2 reads row `row` of w0 and w1.
struct DlRows {
    const uint8_t* w0;  // rows of the matrix (QKV: q, k and v rows stacked in one allocation)
    const uint8_t* w1;  // NG == 2: the second matrix (up)
    uint32_t n_rows;    // output rows of the phase
    uint32_t n_rows4;   // DL_FMT_Q4_TAIL6: rows 0 .. n_rows4 - 1 are w0's (Q4_K), the rest w6's rows (Q6_K)
    const uint8_t* w6;
    uint32_t skip;      // SPREAD phases: leading blocks of the sequence that take no unit (dl_unit)
};

// Issue unit `unit` of a matrix of n_rows rows (Q4_K, or Q6_K with Q6).
template <bool Q6, int NSB, int NG>
__device__ __forceinline__ void dl_issue_unit(DlUnit<NSB, NG>& u, const uint8_t* w0, const uint8_t* w1,
                                              uint32_t n_rows, uint32_t unit) {
    constexpr int BLK = Q6 ? 210 : 144;
    constexpr int ROW_BYTES = NSB * BLK;
    constexpr int RPW = DlUnit<NSB, NG>::RPW;
    const int lane = dl_tid() & 63;
    const int sbo = lane >> 2;
    const int g = lane & 3;
#pragma unroll
    for (int gi = 0; gi < NG; ++gi) {
#pragma unroll
        for (int it = 0; it < DlUnit<NSB, NG>::NIT; ++it) {
            const int sbu = it * 16 + sbo;  // superblock of the unit
            uint32_t row = unit * RPW + (RPW == 1 ? 0 : sbu / NSB);
            row = row < n_rows ? row : n_rows - 1;
            const uint8_t* p = (gi == 0 ? w0 : w1) + (size_t)row * ROW_BYTES + (size_t)(RPW == 1 ? sbu : sbu % NSB) * BLK;
            if constexpr (Q6) {
                // superblocks are 210 B, so only 2-byte aligned: the hardware's unaligned access
                const int h = g >> 1, l0 = (g & 1) * 16;
                u.hdr[gi][it] = load_u4_ua(p + 64 * h + l0);
                u.q0[gi][it] = load_u4_ua(p + 64 * h + 32 + l0);
                u.q1[gi][it] = load_u4_ua(p + 128 + 32 * h + l0);
                u.sc[gi][it] = load_u2_ua(p + 192 + 8 * h);
                u.d[gi][it] = load_u16(p + 208);
            } else {
                u.hdr[gi][it] = load_u4(p);
                u.q0[gi][it] = load_u4(p + 16 + g * 32);
                u.q1[gi][it] = load_u4(p + 32 + g * 32);
            }
        }
    }
}

// Where a phase's input vector comes from.
enum DlSrc {
    DL_SRC_PLAIN = 0,  // fp32, written before the launch (h at layer 0)
    DL_SRC_LL32,       // fp32 + epoch words
    DL_SRC_LL16,       // bf16 + epoch16 words
};

// The old h of the block's rows for a residual epilogue: thread t < 8 upw rpw
// fetches row r = t % rpw of unit (t / rpw) % upw of wave t / (upw rpw) into
// lds[t].
struct DlHold {
    int kind;         // DL_SRC_PLAIN or DL_SRC_LL32; < 0: no residual
    const void* src;
    uint32_t e;
    float* lds;
    int upw;
    int rpw;
    bool spread;      // the phase's unit mapping (dl_unit)
    int nb;           // blocks per sequence (dl_unit's NB: 256 or 64)
    uint32_t n_rows;
    uint64_t* tr;     // phase timeline slots (traced build), else nullptr
};

// Row of hold slot t, or n_rows when the slot's unit has no such row.  Only a
// block's own rows may be read: the phase overwrites every row of h in place,
// each by the block that computes it (reading a row clamped into range would
// race with its owner's overwrite and wait for an epoch that is already gone).
__device__ __forceinline__ uint32_t dl_hold_row(const DlHold& hd, int t) {
    const uint32_t w = (uint32_t)(t / (hd.upw * hd.rpw)), i = (uint32_t)((t / hd.rpw) % hd.upw);
    const uint32_t unit = hd.nb == 64 ? (hd.spread ? dl_unit<true, 64>(w, i) : dl_unit<false, 64>(w, i))
                                      : (hd.spread ? dl_unit<true, 256>(w, i) : dl_unit<false, 256>(w, i));
    const uint32_t row = unit * (uint32_t)hd.rpw + (uint32_t)(t % hd.rpw);
    return row < hd.n_rows ? row : hd.n_rows;
}

// Stage x (K values) in LDS as fp16 pair words + sub-block sums.  RMSNORM:
// x = bf16(h * rsqrt(mean(h^2) + eps) * w); otherwise x = bf16(src).  The
// residual values of the block's rows (hd) are awaited with the same loads.
template <int K, bool RMSNORM>
__device__ __forceinline__ void dl_stage_x(uint32_t* xp, float* xsum, float* xsum16, float* red, int src_kind,
                                           const void* src,
                                           uint32_t e, const float* norm_w, float eps, const DlHold& hd,
                                           uint32_t* status, uint32_t site) {
    // PT float4 per thread; when K does not fill the block, the threads past
    // K/4 in the last step (whole waves, as K % 256 == 0) re-read element 0
    // and stage nothing
    constexpr int PT = (K + 4 * DL_THREADS - 1) / (4 * DL_THREADS);
    constexpr bool FULL = K % (4 * DL_THREADS) == 0;
    static_assert(K % 256 == 0, "K in whole superblocks");
    const int tid = dl_tid();
    auto valid = [&](int j) { return FULL || (j * DL_THREADS + tid) * 4 < K; };
    auto elem = [&](int j) { return valid(j) ? (j * DL_THREADS + tid) * 4 : 0; };
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t hold_row = hd.kind >= 0 && tid < DL_WAVES * hd.upw * hd.rpw ? dl_hold_row(hd, tid) : hd.n_rows;
    const bool has_hold = hold_row < hd.n_rows;
    const uint64_t* hold_ll = reinterpret_cast<const uint64_t*>(hd.src) + hold_row;
    const bool hold_ll_wait = has_hold && hd.kind == DL_SRC_LL32;
    float hold = 0.0f;
    if (has_hold && hd.kind == DL_SRC_PLAIN) hold = reinterpret_cast<const float*>(hd.src)[hold_row];
    float4 hv[PT];
    uint32_t polls = 0;
    if (src_kind == DL_SRC_PLAIN) {
        const float* x = reinterpret_cast<const float*>(src);
#pragma unroll
        for (int j = 0; j < PT; ++j) hv[j] = *reinterpret_cast<const float4*>(x + elem(j));
    } else if (src_kind == DL_SRC_LL32) {
        const uint64_t* x = reinterpret_cast<const uint64_t*>(src);
        uint64_t w[4 * PT];
        polls = ll_wait(w, [&](int i) { return x + elem(i / 4) + (i % 4); },
                        [&](int, uint64_t v) { return ll_ok32(v, e); }, status, site);
#pragma unroll
        for (int j = 0; j < PT; ++j)
            hv[j] = make_float4(ll_val32(w[4 * j]), ll_val32(w[4 * j + 1]), ll_val32(w[4 * j + 2]),
                                ll_val32(w[4 * j + 3]));
    } else {
        // 2 elements per word; word 2 PT is the residual value (threads without one re-read word 0)
        const uint64_t* x = reinterpret_cast<const uint64_t*>(src);
        uint64_t w[2 * PT + 1];
        polls = ll_wait(w,
                [&](int i) {
                    return i < 2 * PT ? x + elem(i / 2) / 2 + (i % 2) : (hold_ll_wait ? hold_ll : x + elem(0) / 2);
                },
                [&](int i, uint64_t v) {
                    return i < 2 * PT || !hold_ll_wait ? ll_ok16x2(v, e) : ll_ok32(v, hd.e);
                },
                status, site);
#pragma unroll
        for (int j = 0; j < PT; ++j)
            hv[j] = make_float4(bf16_bits_to_f32((uint32_t)w[2 * j] & 0xffffu),
                                bf16_bits_to_f32((uint32_t)(w[2 * j] >> 32) & 0xffffu),
                                bf16_bits_to_f32((uint32_t)w[2 * j + 1] & 0xffffu),
                                bf16_bits_to_f32((uint32_t)(w[2 * j + 1] >> 32) & 0xffffu));
        if (hold_ll_wait) hold = ll_val32(w[2 * PT]);
    }
    if (hd.tr != nullptr && tid == 0) hd.tr[DL_TR_POLLS] = polls;
    if (has_hold) hd.lds[tid] = hold;
#pragma unroll
    for (int j = 0; j < PT; ++j)
        if (!valid(j)) hv[j] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if constexpr (RMSNORM) {
        // (loading the norm weights before the input wait instead measured slower for both shapes)
        float4 wv[PT];
#pragma unroll
        for (int j = 0; j < PT; ++j) wv[j] = *reinterpret_cast<const float4*>(norm_w + elem(j));
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
            if (!valid(j)) continue;
            const int k = (j * DL_THREADS + tid) * 4;
            stage_x4(xp, xsum, k, bf16_round(hv[j].x * inv * wv[j].x), bf16_round(hv[j].y * inv * wv[j].y),
                     bf16_round(hv[j].z * inv * wv[j].z), bf16_round(hv[j].w * inv * wv[j].w), xsum16);
        }
    } else {
#pragma unroll
        for (int j = 0; j < PT; ++j) {
            if (!valid(j)) continue;
            const int k = (j * DL_THREADS + tid) * 4;
            stage_x4(xp, xsum, k, bf16_round(hv[j].x), bf16_round(hv[j].y), bf16_round(hv[j].z),
                     bf16_round(hv[j].w), xsum16);
        }
    }
    __syncthreads();
}

enum DlEpi { DL_EPI_STORE = 0, DL_EPI_RESID = 1, DL_EPI_SWIGLU = 2 };

// Wave-reduced dot products of one unit against the staged x, one x slice
// live at a time.
template <int NSB, int NG>
__device__ __forceinline__ void dl_dot_unit(const DlUnit<NSB, NG>& u, const uint32_t* xp, const float* xsum,
                                            const Q4LaneConsts& lc, float (&res)[NG][DlUnit<NSB, NG>::RPW]) {
    constexpr int NIT = DlUnit<NSB, NG>::NIT;
    constexpr int RPW = DlUnit<NSB, NG>::RPW;
    const int lane = dl_tid() & 63;
    const int sbo = lane >> 2;
    const int g = lane & 3;
    float acc[NG][RPW];
#pragma unroll
    for (int it = 0; it < NIT; ++it) {
        const int sbu = it * 16 + sbo;
        XSlice16 xs;
        load_xslice16(xp, xsum, RPW == 1 ? sbu : sbu % NSB, g, xs);
#pragma unroll
        for (int gi = 0; gi < NG; ++gi) {
            const float c = q4k_lane_dot(u.hdr[gi][it], u.q0[gi][it], u.q1[gi][it], xs, lc);
            if constexpr (RPW == 1) {
                acc[gi][0] = it == 0 ? c : acc[gi][0] + c;
            } else {
#pragma unroll
                for (int r = 0; r < RPW; ++r) {
                    const float v = sbu / NSB == r ? c : 0.0f;
                    acc[gi][r] = it == 0 ? v : acc[gi][r] + v;
                }
            }
        }
    }
#pragma unroll
    for (int gi = 0; gi < NG; ++gi)
#pragma unroll
        for (int r = 0; r < RPW; ++r) res[gi][r] = wave_sum(acc[gi][r]);
}

// The same for a Q6_K unit.  A lane's piece is 16 values of each of 4 parts
// (values 32 p + l0 .. + 15 of half h): each run is 8 pair words of the staged
// x.  Codes q (6 bits) become fp16 1024 + q with one and-or, so
//   sum x (q - 32) = sum x (1024 + q) - 1056 sum x,
// the second sum from the staged 16-value sums.
// Q6_K: value(128h + 32p + l) = d * sc[8h + 2p + l/16] * (q - 32),
//   q = (ql[64h + 32(p&1) + l] >> 4(p>>1) & 15) | ((qh[32h + l] >> 2p) & 3) << 4.
template <int NSB, int NG>
__device__ __forceinline__ void dl_dot_unit6(const DlUnit<NSB, NG>& u, const uint32_t* xp, const float* xsum16,
                                             float (&res)[NG][DlUnit<NSB, NG>::RPW]) {
    constexpr int NIT = DlUnit<NSB, NG>::NIT;
    constexpr int RPW = DlUnit<NSB, NG>::RPW;
    constexpr uint32_t B = 0x64006400u, LO = 0x000f000fu, HI = 0x00300030u;
    const int lane = dl_tid() & 63;
    const int sbo = lane >> 2;
    const int g = lane & 3;
    const int h = g >> 1, l0 = (g & 1) * 16, sh = (g & 1) * 8;
    float acc[NG][RPW];
#pragma unroll
    for (int it = 0; it < NIT; ++it) {
        const int sbu = it * 16 + sbo;
        const int e0 = (RPW == 1 ? sbu : sbu % NSB) * 256 + 128 * h + l0;  // first value of part 0
        uint32_t x[4][8];
        float xs[4];
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            const uint32_t* xw = xp + xp_word(e0 + 32 * p);
            const uint4 a = *reinterpret_cast<const uint4*>(xw);
            const uint4 b = *reinterpret_cast<const uint4*>(xw + 4);
            x[p][0] = a.x; x[p][1] = a.y; x[p][2] = a.z; x[p][3] = a.w;
            x[p][4] = b.x; x[p][5] = b.y; x[p][6] = b.z; x[p][7] = b.w;
            xs[p] = xsum16[(e0 + 32 * p) >> 4];
        }
#pragma unroll
        for (int gi = 0; gi < NG; ++gi) {
            const uint4 qa = u.hdr[gi][it], qb = u.q0[gi][it], qc = u.q1[gi][it];
            const uint32_t ql0[4] = {qa.x, qa.y, qa.z, qa.w};
            const uint32_t ql1[4] = {qb.x, qb.y, qb.z, qb.w};
            const uint32_t qh[4] = {qc.x, qc.y, qc.z, qc.w};
            float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f, s3 = 0.0f;
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const uint32_t w0 = ql0[c], w1 = ql1[c], hq = qh[c];
                s0 = dot2_f16((w0 & LO) | ((hq << 4) & HI) | B, x[0][2 * c], s0);
                s0 = dot2_f16(((w0 >> 8) & LO) | ((hq >> 4) & HI) | B, x[0][2 * c + 1], s0);
                s1 = dot2_f16((w1 & LO) | ((hq << 2) & HI) | B, x[1][2 * c], s1);
                s1 = dot2_f16(((w1 >> 8) & LO) | ((hq >> 6) & HI) | B, x[1][2 * c + 1], s1);
                s2 = dot2_f16(((w0 >> 4) & LO) | (hq & HI) | B, x[2][2 * c], s2);
                s2 = dot2_f16(((w0 >> 12) & LO) | ((hq >> 8) & HI) | B, x[2][2 * c + 1], s2);
                s3 = dot2_f16(((w1 >> 4) & LO) | ((hq >> 2) & HI) | B, x[3][2 * c], s3);
                s3 = dot2_f16(((w1 >> 12) & LO) | ((hq >> 10) & HI) | B, x[3][2 * c + 1], s3);
            }
            // int8 scales sc[8h + 2p + l0 / 16]: byte (l0 / 16) and 2 + (l0 / 16) of each dword
            const uint2 scw = u.sc[gi][it];
            const float sc0 = (float)(int8_t)((scw.x >> sh) & 0xffu);
            const float sc1 = (float)(int8_t)((scw.x >> (16 + sh)) & 0xffu);
            const float sc2 = (float)(int8_t)((scw.y >> sh) & 0xffu);
            const float sc3 = (float)(int8_t)((scw.y >> (16 + sh)) & 0xffu);
            float t = sc0 * fmaf(-1056.0f, xs[0], s0);
            t = fmaf(sc1, fmaf(-1056.0f, xs[1], s1), t);
            t = fmaf(sc2, fmaf(-1056.0f, xs[2], s2), t);
            t = fmaf(sc3, fmaf(-1056.0f, xs[3], s3), t);
            const float c = f16_bits_to_f32(u.d[gi][it] & 0xffffu) * t;
            if constexpr (RPW == 1) {
                acc[gi][0] = it == 0 ? c : acc[gi][0] + c;
            } else {
#pragma unroll
                for (int r = 0; r < RPW; ++r) {
                    const float v = sbu / NSB == r ? c : 0.0f;
                    acc[gi][r] = it == 0 ? v : acc[gi][r] + v;
                }
            }
        }
    }
#pragma unroll
    for (int gi = 0; gi < NG; ++gi)
#pragma unroll
        for (int r = 0; r < RPW; ++r) res[gi][r] = wave_sum(acc[gi][r]);
}

// Where a phase's output goes.
struct DlOut {
    uint64_t* ll32;      // STORE / RESID: fp32 + epoch words
    uint32_t* ll16;      // SWIGLU: bf16 + epoch16 words
    float* plain;        // RESID on the last layer: the caller's h (no epoch)
    DlHold hold;         // RESID: where the old h comes from (staged in LDS with x)
    uint32_t e_out;      // epoch written
    uint64_t* tr;        // phase timeline slots (traced build), else nullptr
};

//   STORE: y[row] = dot;  RESID: y[row] = h_old[row] + dot;  SWIGLU: y[row] = bf16(silu(g) * u)
// for the RPW rows of one unit.
template <int NG, int RPW, int EPI>
__device__ __forceinline__ void dl_store_unit(const DlOut& o, uint32_t unit, uint32_t n_rows,
                                              const float (&res)[NG][RPW], const float* hold) {
    if ((dl_tid() & 63) == 0) {
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
            const uint32_t row = unit * RPW + r;
            if (row >= n_rows) break;
            if constexpr (EPI == DL_EPI_STORE) {
                ll_put32(o.ll32 + row, res[0][r], o.e_out);
            } else if constexpr (EPI == DL_EPI_RESID) {
                const float old = hold[r];
                if (o.plain != nullptr)
                    o.plain[row] = old + res[0][r];
                else
                    ll_put32(o.ll32 + row, old + res[0][r], o.e_out);
            } else {
                ll_put16(o.ll16 + row, silu(res[0][r]) * res[NG - 1][r], o.e_out);
            }
        }
    }
}

// Issue unit slot i of the wave (unit dl_unit<SPREAD>(wave, i)) in the phase's
// format.  DL_FMT_Q4_TAIL6: units from n_rows4 / RPW on are Q6_K units of w6;
// only the last slot can hold one (units grow with the slot), so the others
// are Q4_K at compile time.
template <int FMT, int UPW, bool SPREAD, int NB, int NSB, int NG>
__device__ __forceinline__ void dl_issue_slot(DlUnit<NSB, NG>& u, const DlRows& r, int wave, int i) {
    constexpr int RPW = DlUnit<NSB, NG>::RPW;
    const uint32_t unit = dl_unit<SPREAD, NB>(wave, i, r.skip);
    if constexpr (FMT == DL_FMT_Q6) {
        dl_issue_unit<true>(u, r.w0, r.w1, r.n_rows, unit);
    } else if constexpr (FMT == DL_FMT_Q4_TAIL6) {
        const uint32_t units4 = r.n_rows4 / RPW;
        if (i == UPW - 1 && unit >= units4)
            dl_issue_unit<true>(u, r.w6, r.w6, r.n_rows - r.n_rows4, unit - units4);
        else
            dl_issue_unit<false>(u, r.w0, r.w1, r.n_rows4, unit);
    } else {
        dl_issue_unit<false>(u, r.w0, r.w1, r.n_rows, unit);
    }
}

// The first PRE units of a GEMV phase.  SPREAD phases: waves without a unit
// issue nothing.
template <int NSB, int NG, int UPW, int PRE, bool SPREAD, int NB, int FMT = DL_FMT_Q4>
__device__ __forceinline__ void dl_issue_pre(DlUnit<NSB, NG> (&u)[UPW], const DlRows& rows) {
    constexpr int RPW = DlUnit<NSB, NG>::RPW;
    const int wave = __builtin_amdgcn_readfirstlane(dl_tid() >> 6);
    if (SPREAD && dl_unit<SPREAD, NB>(wave, 0, rows.skip) >= (rows.n_rows + RPW - 1) / RPW) return;
#pragma unroll
    for (int i = 0; i < PRE; ++i) dl_issue_slot<FMT, UPW, SPREAD, NB>(u[i], rows, wave, i);
}

// One GEMV phase over the wave's UPW units (rows wrow + i * DL_NW), streamed
// through a ring of R units whose first PRE the caller issued (dl_issue_pre)
// before the phase's input is awaited: they stream during the hand-off, and
// the wait queues behind them, so PRE trades HBM occupancy at the phase
// boundary against input latency.  Once the input is staged, units PRE .. R-1
// are issued, then unit i + R right after unit i has been reduced.  The loop
// is unrolled, so the ring is static registers, and the scheduling fences
// keep each refill after the reduction that frees its registers.
// SPREAD: fewer units than waves (dl_unit); a wave without a unit issues and
// stores nothing.  FMT: the units' weight formats (DlFmt).
template <int NSB, int NG, int UPW, int R, int PRE, int EPI, bool RMSNORM, bool SPREAD, int FMT = DL_FMT_Q4,
          class SH, class Hook = DlNoHook, int NB = SH::NB>
__device__ __forceinline__ void dl_gemv_phase(SH& sm, DlUnit<NSB, NG> (&u)[UPW], const DlRows& rows, int src_kind,
                                              const void* x_src, uint32_t e_x, const float* norm_w, float eps,
                                              const DlOut& out, uint32_t* status, uint32_t site,
                                              Hook after_issue = Hook()) {
    static_assert(PRE >= 0 && PRE <= R && R >= 1 && R <= UPW, "ring size");
    constexpr int RPW = DlUnit<NSB, NG>::RPW;
    static_assert(EPI != DL_EPI_RESID || UPW * RPW <= DL_HOLD, "residual rows per wave");
    static_assert(!SPREAD || UPW == 1, "spread phases have one unit per wave");
    const int wave = __builtin_amdgcn_readfirstlane(dl_tid() >> 6);
    const uint32_t n_units = (rows.n_rows + RPW - 1) / RPW;
    const bool active = !SPREAD || dl_unit<SPREAD, NB>(wave, 0, rows.skip) < n_units;  // wave-uniform
    __syncthreads();  // every wave is done with the previous phase's LDS
    DlHold hd = out.hold;
    hd.lds = sm.g.hold;
    hd.upw = UPW;
    hd.rpw = RPW;
    hd.spread = SPREAD;
    hd.nb = NB;
    hd.n_rows = rows.n_rows;
    hd.tr = out.tr;
    if (EPI != DL_EPI_RESID) hd.kind = -1;
    dl_stage_x<NSB * 256, RMSNORM>(sm.g.xp, sm.g.xsum, FMT == DL_FMT_Q4 ? nullptr : sm.g.xsum16, sm.g.red, src_kind,
                                   x_src, e_x, norm_w, eps, hd, status, site);
    dl_stamp(out.tr, DL_TR_READY);
    // after_issue: the caller's early loads for the next phase, right behind this phase's last unit (every
    // wave calls it once, with or without units)
    if (!active) {
        after_issue();
        return;
    }
#pragma unroll
    for (int i = PRE; i < R; ++i) dl_issue_slot<FMT, UPW, SPREAD, NB>(u[i], rows, wave, i);
    if constexpr (R >= UPW) after_issue();
    const Q4LaneConsts lc = q4k_lane_consts(dl_tid() & 3);
#pragma unroll
    for (int i = 0; i < UPW; ++i) {
        __builtin_amdgcn_sched_barrier(0);
        float res[NG][RPW];
        const uint32_t unit = dl_unit<SPREAD, NB>(wave, i, rows.skip);
        if constexpr (FMT == DL_FMT_Q6) {
            dl_dot_unit6(u[i], sm.g.xp, sm.g.xsum16, res);
        } else if constexpr (FMT == DL_FMT_Q4_TAIL6) {
            if (i == UPW - 1 && unit >= rows.n_rows4 / RPW)
                dl_dot_unit6(u[i], sm.g.xp, sm.g.xsum16, res);
            else
                dl_dot_unit(u[i], sm.g.xp, sm.g.xsum, lc, res);
        } else {
            dl_dot_unit(u[i], sm.g.xp, sm.g.xsum, lc, res);
        }
        if (i == 0) dl_stamp(out.tr, DL_TR_FIRST);
        dl_store_unit<NG, RPW, EPI>(out, unit, rows.n_rows, res, &sm.g.hold[(wave * UPW + i) * RPW]);
        __builtin_amdgcn_sched_barrier(0);
        if (i + R < UPW) dl_issue_slot<FMT, UPW, SPREAD, NB>(u[i + R], rows, wave, i + R);
        if (i + R == UPW - 1) after_issue();
    }
}

// --------------------------------------------------------- attention phase ----

// K and V rows of one wave's 32 positions, loaded ahead of the scores.
// K is the A operand of v_mfma_f32_16x16x32_bf16 (lane l: row l % 16 of a
// 16-position tile, dims 32 c + 8 (l / 16) .. + 7 of chunk c); tile t row r is
// position 8 (r / 4) + 4 t + r % 4, so that a lane's 8 scores come out as the
// positions 8 (l / 16) .. + 7.  V: lane l holds dims 8 (l % 16) .. + 7 of those
// same positions, for P.V on the VALU.
struct DlAttnBank {
    uint4 kr[2][4];
    uint4 vr[8];
};

__device__ __forceinline__ int dl_att_kpos(int lane, int t) {
    const int r = lane & 15;
    return 8 * (r >> 2) + 4 * t + (r & 3);
}

template <int SLOTS>
__device__ __forceinline__ int dl_att_span(int L) {
    // positions per wave: the kv head's L positions over its SLOTS * DL_WAVES waves
    return (L + SLOTS * DL_WAVES - 1) / (SLOTS * DL_WAVES);
}

// Positions of the wave's span it covers: rows = clamp(L - p0, 0, span).
__device__ __forceinline__ int dl_att_rows(int L, int p0, int span) {
    const int rows = L - p0;
    return rows < 0 ? 0 : (rows > span ? span : rows);
}

// Only the wave's own rows are loaded (rows of a short span would otherwise be
// the next wave's, fetched twice); the registers of the others are zero, so
// that P = 0 times V stays 0.
__device__ __forceinline__ void dl_attn_issue_k(DlAttnBank& bk, const uint16_t* kc, int kvh, int p0, int rows) {
    const int lane = dl_tid() & 63;
    const int kg = lane >> 4;
    const size_t stride = (size_t)8 * DL_D;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        const int p = dl_att_kpos(lane, t);
        const bool in = p < rows;
        const uint16_t* row = kc + (size_t)(in ? p0 + p : 0) * stride + (size_t)kvh * DL_D + 8 * kg;
#pragma unroll
        for (int c = 0; c < 4; ++c) bk.kr[t][c] = in ? load_u4(row + 32 * c) : make_uint4(0u, 0u, 0u, 0u);
    }
}

__device__ __forceinline__ void dl_attn_issue_v(DlAttnBank& bk, const uint16_t* vc, int kvh, int p0, int rows) {
    const int lane = dl_tid() & 63;
    const int part = lane & 15, pg = lane >> 4;
    const size_t stride = (size_t)8 * DL_D;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const bool in = 8 * pg + j < rows;
        const uint16_t* row = vc + (size_t)(in ? p0 + 8 * pg + j : 0) * stride + (size_t)kvh * DL_D + part * 8;
        bk.vr[j] = in ? load_u4(row) : make_uint4(0u, 0u, 0u, 0u);
    }
}

// Per-head RMSNorm (weights w0, w1 of the lane's dims lane and lane + 64, loaded by the caller before its
// input wait) and rotate-half RoPE.
__device__ __forceinline__ void dl_norm_rope(float x0, float x1, float w0, float w1, bool has_w, float eps, float cs,
                                             float sn, bool rope, float& r0, float& r1) {
    float n0 = x0, n1 = x1;
    if (has_w) {
        const float ss = wave_sum(x0 * x0 + x1 * x1);
        const float inv = 1.0f / sqrtf(ss / (float)DL_D + eps);
        n0 = x0 * inv * w0;
        n1 = x1 * inv * w1;
    }
    if (rope) {
        r0 = n0 * cs - n1 * sn;
        r1 = n1 * cs + n0 * sn;
    } else {
        r0 = n0;
        r1 = n1;
    }
}

// Block (kv head kvh, slot bs): the wave covers positions [p0, p0 + rows).  The
// block's (max, sum, output) per q head goes to part[kvh][bs]; with `direct` (the
// block covers every position of its kv head) the normalised output goes to the
// attention output words instead, with epoch e_out either way.
template <class S, class Hook = DlNoHook>
__device__ __forceinline__ void dl_attn_phase(DlAttnBank& bk, DlAttnLds<S::GROUP, S::pv_mfma>& sm, const DlArgs& a,
                                              const uint64_t* lp, int kvh, int bs, int p0, int rows, bool direct,
                                              int pos, float cs, float sn, uint32_t e_qkv, uint32_t e_out,
                                              uint32_t site, uint64_t* tr, Hook after_ready = Hook()) {
    constexpr int GROUP = S::GROUP;
    const int tid = dl_tid(), lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int s_cap = (int)a.s_cap;
    const bool has_new = pos < s_cap && pos >= p0 && pos < p0 + rows;
    const int rnew = pos - p0;
    const bool rope = a.theta > 0.0f;
    const float* q_norm = dl_gptr<const float>(lp[DL_Q_NORM]);
    const float* k_norm = dl_gptr<const float>(lp[DL_K_NORM]);
    uint16_t* kc = dl_gptr<uint16_t>(lp[DL_K_CACHE]);
    uint16_t* vc = dl_gptr<uint16_t>(lp[DL_V_CACHE]);
    const uint64_t* q = a.qkv_ll;
    const uint64_t* kn = a.qkv_ll + S::QD;
    const uint64_t* vn = a.qkv_ll + S::QD + S::KVD;
    auto ok = [&](int, uint64_t v) { return ll_ok32(v, e_qkv); };
    // the q / k norm weights of the lane's dims, in flight before the waits below
    const bool q_wave = wave < GROUP;
    float qw0 = 1.0f, qw1 = 1.0f, kw0 = 1.0f, kw1 = 1.0f;
    if (q_wave && q_norm != nullptr) {
        qw0 = q_norm[lane];
        qw1 = q_norm[lane + 64];
    }
    if (has_new && k_norm != nullptr) {
        kw0 = k_norm[lane];
        kw1 = k_norm[lane + 64];
    }
    __syncthreads();  // every wave is done with the previous phase's LDS

    if (q_wave) {
        const int hq = kvh * GROUP + wave;
        uint64_t w[2];
        const uint32_t polls =
            ll_wait(w, [&](int i) { return q + hq * DL_D + lane + 64 * i; }, ok, a.status, site | DL_W_ATTN_Q);
        if (tr != nullptr && tid == 0) tr[DL_TR_POLLS] = polls;
        float r0, r1;
        dl_norm_rope(ll_val32(w[0]), ll_val32(w[1]), qw0, qw1, q_norm != nullptr, a.eps, cs, sn, rope, r0, r1);
        // scores in base-2 units (log2(e) / sqrt(D) folded into q): the softmax and every combine of partials
        // below are exp2 of differences, one v_exp_f32 each
        const float scale = 1.4426950408889634f / sqrtf((float)DL_D);
        const float q0 = r0 * scale, q1 = r1 * scale;
        const uint32_t h0 = f32_to_bf16_bits(q0), h1 = f32_to_bf16_bits(q1);
        sm.qhi[wave][lane] = (uint16_t)h0;
        sm.qhi[wave][lane + 64] = (uint16_t)h1;
        sm.qlo[wave][lane] = (uint16_t)f32_to_bf16_bits(q0 - bf16_bits_to_f32(h0));
        sm.qlo[wave][lane + 64] = (uint16_t)f32_to_bf16_bits(q1 - bf16_bits_to_f32(h1));
    }
    uint32_t vnew = 0;
    if (has_new) {
        uint64_t w[4];
        ll_wait(w, [&](int i) { return i < 2 ? kn + kvh * DL_D + lane + 64 * i : vn + kvh * DL_D + 2 * lane + (i - 2); },
                ok, a.status, site | DL_W_ATTN_KV);
        float k0, k1;
        dl_norm_rope(ll_val32(w[0]), ll_val32(w[1]), kw0, kw1, k_norm != nullptr, a.eps, cs, sn, rope, k0, k1);
        const uint16_t kb0 = (uint16_t)f32_to_bf16_bits(k0), kb1 = (uint16_t)f32_to_bf16_bits(k1);
        sm.knew[lane] = kb0;
        sm.knew[lane + 64] = kb1;
        vnew = pack_bf16x2(ll_val32(w[2]), ll_val32(w[3]));
        reinterpret_cast<uint32_t*>(sm.vnew)[lane] = vnew;
        const size_t off = (size_t)pos * 8 * DL_D + (size_t)kvh * DL_D;
        kc[off + lane] = kb0;
        kc[off + lane + 64] = kb1;
        reinterpret_cast<uint32_t*>(vc + off)[lane] = vnew;
    }
    __syncthreads();
    dl_stamp(tr, DL_TR_READY);
    if constexpr (!S::o_late) after_ready();

    // Scores S[position][head] = K . q^T on the matrix cores: two 16-position
    // tiles, 4 chunks of 32 dims, q as bf16 hi + lo (columns >= GROUP are 0).
    // Lane l then holds head l % 16 at positions 8 (l / 16) + 4 t + i.
    const int kg = lane >> 4, n = lane & 15;
    const int pg = kg, part = n;  // the P.V view of the same lane
    dl_bf16x8_t qh[4], ql[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        uint4 h = make_uint4(0u, 0u, 0u, 0u), lo = h;
        if (n < GROUP) {
            h = *reinterpret_cast<const uint4*>(&sm.qhi[n][32 * c + 8 * kg]);
            lo = *reinterpret_cast<const uint4*>(&sm.qlo[n][32 * c + 8 * kg]);
        }
        qh[c] = __builtin_bit_cast(dl_bf16x8_t, h);
        ql[c] = __builtin_bit_cast(dl_bf16x8_t, lo);
    }
    // the new position's row: read from LDS into registers first and selected as a value (a select between
    // two loads would be merged into one generic load through a selected pointer, re-reading the cache row)
    uint4 knr[4] = {}, vnr = {};
    if (has_new) {
#pragma unroll
        for (int c = 0; c < 4; ++c) knr[c] = *reinterpret_cast<const uint4*>(&sm.knew[32 * c + 8 * kg]);
        vnr = *reinterpret_cast<const uint4*>(&sm.vnew[part * 8]);
    }
    dl_f32x4_t acc[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        const bool sub = has_new && dl_att_kpos(lane, t) == rnew;
        acc[t] = dl_f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const uint4 kk = sub ? knr[c] : bk.kr[t][c];
            const dl_bf16x8_t ka = __builtin_bit_cast(dl_bf16x8_t, kk);
            acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka, qh[c], acc[t], 0, 0, 0);
            acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka, ql[c], acc[t], 0, 0, 0);
        }
    }
    if constexpr (S::o_late) after_ready();
    if (tr != nullptr) dl_stamp(tr, DL_TR_A_SCORES);
    // softmax of head n over the wave's positions (the 4 lanes n, 16 + n, 32 + n, 48 + n)
    float sc[8];
    bool valid[8];
    float m = -INFINITY;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        sc[j] = acc[j >> 2][j & 3];
        valid[j] = 8 * kg + j < rows;
        m = fmaxf(m, valid[j] ? sc[j] : -INFINITY);
    }
    m = xor_max<16>(m);
    m = xor_max<32>(m);
    float e[8];
    float l = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        e[j] = valid[j] ? __builtin_amdgcn_exp2f(sc[j] - m) : 0.0f;
        l += e[j];
    }
    l = xor_sum<16>(l);
    l = xor_sum<32>(l);
    dl_stamp(tr, DL_TR_FIRST);
    if constexpr (S::pv_mfma) {
        // P.V on the matrix cores: O[head][dim] = P[head][position] . V[position][dim].  P is the A operand as the
        // scores left it (lane l: head l % 16 at positions 8 (l / 16) + j), as bf16 hi + lo; V goes through LDS:
        // the wave's rows are stored [position][dims] and read back transposed, lane 4 j + q of row group g
        // addressing row 8 g + j (+ 4), dims 16 T + 4 q, so that lane i of the group receives dim 16 T + i of
        // positions 8 g + 0..7, the B operand of dim tile T.
        uint16_t* vs = sm.vst[wave];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint4 vv = (has_new && rnew == 8 * pg + j) ? vnr : bk.vr[j];
            *reinterpret_cast<uint4*>(vs + (8 * pg + j) * DL_VROW + part * 8) = vv;
        }
        uint4 ph4, pl4;
        {
            uint32_t hb[8], lb[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                hb[j] = f32_to_bf16_bits(e[j]);
                lb[j] = f32_to_bf16_bits(e[j] - bf16_bits_to_f32(hb[j]));
            }
            ph4 = make_uint4(hb[0] | hb[1] << 16, hb[2] | hb[3] << 16, hb[4] | hb[5] << 16, hb[6] | hb[7] << 16);
            pl4 = make_uint4(lb[0] | lb[1] << 16, lb[2] | lb[3] << 16, lb[4] | lb[5] << 16, lb[6] | lb[7] << 16);
        }
        const dl_bf16x8_t pa_hi = __builtin_bit_cast(dl_bf16x8_t, ph4), pa_lo = __builtin_bit_cast(dl_bf16x8_t, pl4);
        const uint16_t* vt = vs + (8 * kg + (n >> 2)) * DL_VROW + 4 * (n & 3);
        dl_f32x4_t ov[DL_D / 16];
#pragma unroll
        for (int t = 0; t < DL_D / 16; ++t) {
            const uint2 b0 = lds_read_tr16_b64(vt + 16 * t);
            const uint2 b1 = lds_read_tr16_b64(vt + 4 * DL_VROW + 16 * t);
            const dl_bf16x8_t vb = __builtin_bit_cast(dl_bf16x8_t, make_uint4(b0.x, b0.y, b1.x, b1.y));
            ov[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pa_hi, vb, dl_f32x4_t{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
            ov[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pa_lo, vb, ov[t], 0, 0, 0);
        }
        if (tr != nullptr) dl_stamp(tr, DL_TR_A_PV);
        // lanes 0..15 hold heads 0..3 of dims 16 T + lane
        if (lane < 16) {
#pragma unroll
            for (int t = 0; t < DL_D / 16; ++t)
                sm.wo[wave][16 * t + lane] = make_float4(ov[t][0], ov[t][1], ov[t][2], ov[t][3]);
        }
    } else {
        // P of every head at the row's 8 positions, from lanes 0 .. GROUP-1 of the row (row_newbcast)
        constexpr int NV = GROUP * 8;
        float p[NV];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            p[0 * 8 + j] = dpp_f32<0x150>(e[j]);
            p[1 * 8 + j] = dpp_f32<0x151>(e[j]);
            if constexpr (GROUP == 4) {
                p[2 * 8 + j] = dpp_f32<0x152>(e[j]);
                p[3 * 8 + j] = dpp_f32<0x153>(e[j]);
            }
        }
        // P.V over the row's positions (dims 8 part .. + 7), then summed over the 4 rows (scattered)
        float o[NV];
#pragma unroll
        for (int i = 0; i < NV; ++i) o[i] = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint4 vv = (has_new && rnew == 8 * pg + j) ? vnr : bk.vr[j];
            const float vf[8] = {bf16_bits_to_f32(vv.x & 0xffffu), bf16_bits_to_f32(vv.x >> 16),
                                 bf16_bits_to_f32(vv.y & 0xffffu), bf16_bits_to_f32(vv.y >> 16),
                                 bf16_bits_to_f32(vv.z & 0xffffu), bf16_bits_to_f32(vv.z >> 16),
                                 bf16_bits_to_f32(vv.w & 0xffffu), bf16_bits_to_f32(vv.w >> 16)};
#pragma unroll
            for (int gg = 0; gg < GROUP; ++gg)
#pragma unroll
                for (int d = 0; d < 8; ++d) o[gg * 8 + d] = fmaf(p[gg * 8 + j], vf[d], o[gg * 8 + d]);
        }
        // reduce-scatter over the 4 rows: lanes with bit 5 (then 4) clear keep the lower half, each adding its
        // partner's partial of that half
        float o1[NV / 2], of[NV / 4];
#pragma unroll
        for (int i = 0; i < NV / 2; ++i) o1[i] = xor_reduce_scatter<32>(o[i], o[NV / 2 + i]);
#pragma unroll
        for (int i = 0; i < NV / 4; ++i) of[i] = xor_reduce_scatter<16>(o1[i], o1[NV / 4 + i]);
        if (tr != nullptr) dl_stamp(tr, DL_TR_A_PV);
        // the lane holds head og, dims 8 part + od .. + NV/4 - 1
        const int obase = (pg >> 1) * (NV / 2) + (pg & 1) * (NV / 4);
        const int og = obase / 8, od = obase % 8;
        float* wo = reinterpret_cast<float*>(&sm.wo[wave][0]) + og * DL_D + part * 8 + od;
#pragma unroll
        for (int i = 0; i < NV / 4; ++i) wo[i] = of[i];
    }
    if (kg == 0 && n < GROUP) {
        sm.wml[wave][n][0] = m;
        sm.wml[wave][n][1] = l;
    }
    __syncthreads();
    if (tr != nullptr) dl_stamp(tr, DL_TR_A_MERGED);
    // block partial: [kvh][bs][g] = (M, l, o[128])
    uint64_t* pb = a.part_ll + (((size_t)kvh * S::ATT_SLOTS + bs) * GROUP) * (2 + DL_D);
    for (int idx = tid; idx < GROUP * 64; idx += DL_THREADS) {
        const int gg = idx >> 6, dl = idx & 63;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < DL_WAVES; ++w) M = fmaxf(M, sm.wml[w][gg][0]);
        float l = 0.0f, r0 = 0.0f, r1 = 0.0f;
#pragma unroll
        for (int w = 0; w < DL_WAVES; ++w) {
            const float m = sm.wml[w][gg][0];
            const float f = m == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m - M);
            l = fmaf(f, sm.wml[w][gg][1], l);
            float2 ov;
            if constexpr (S::pv_mfma)
                ov = make_float2(reinterpret_cast<const float*>(&sm.wo[w][2 * dl])[gg],
                                 reinterpret_cast<const float*>(&sm.wo[w][2 * dl + 1])[gg]);
            else
                ov = reinterpret_cast<const float2*>(reinterpret_cast<const float*>(&sm.wo[w][0]) + gg * DL_D)[dl];
            r0 = fmaf(f, ov.x, r0);
            r1 = fmaf(f, ov.y, r1);
        }
        if (direct) {
            const float inv = 1.0f / l;
            ll_store(reinterpret_cast<uint64_t*>(a.attn_ll) + ((kvh * GROUP + gg) * DL_D) / 2 + dl,
                     ll_pack16x2(r0 * inv, r1 * inv, e_out));
            continue;
        }
        uint64_t* pg = pb + gg * (2 + DL_D);
        ll_put32(pg + 2 + 2 * dl, r0, e_out);
        ll_put32(pg + 3 + 2 * dl, r1, e_out);
        if (dl == 0) {
            ll_put32(pg, M, e_out);
            ll_put32(pg + 1, l, e_out);
        }
    }
}

// Head hq (< NH): merge the S::ATT_SLOTS block partials of its kv head.
template <class S>
__device__ __forceinline__ void dl_merge_phase(DlAttnLds<S::GROUP, S::pv_mfma>& sm, const DlArgs& a, int hq,
                                               uint32_t e_part, uint32_t e_attn, uint32_t site, uint64_t* tr) {
    constexpr int GROUP = S::GROUP;
    const int tid = dl_tid(), lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int kvh = hq / GROUP, gg = hq % GROUP;
    constexpr int PER_WAVE = S::ATT_SLOTS / DL_WAVES;  // partials per wave: 4 (1 with 64 blocks per sequence)
    __syncthreads();  // every wave is done with the previous phase's LDS
    uint64_t w[4 * PER_WAVE];
    const uint32_t polls = ll_wait(w, [&](int i) {
                const int bs = wave * PER_WAVE + i / 4, k = i % 4;
                const uint64_t* pg = a.part_ll + (((size_t)kvh * S::ATT_SLOTS + bs) * GROUP + gg) * (2 + DL_D);
                return k < 2 ? pg + k : pg + 2 + 2 * lane + (k - 2);
            },
            [&](int, uint64_t v) { return ll_ok32(v, e_part); }, a.status, site | DL_W_MERGE);
    if (tr != nullptr && tid == 0) tr[DL_TR_POLLS] = polls;
    dl_stamp(tr, DL_TR_READY);
    float2 ml[PER_WAVE], ov[PER_WAVE];
#pragma unroll
    for (int i = 0; i < PER_WAVE; ++i) {
        ml[i] = make_float2(ll_val32(w[4 * i]), ll_val32(w[4 * i + 1]));
        ov[i] = make_float2(ll_val32(w[4 * i + 2]), ll_val32(w[4 * i + 3]));
    }
    float M = -INFINITY;
#pragma unroll
    for (int i = 0; i < PER_WAVE; ++i) M = fmaxf(M, ml[i].x);
    float l = 0.0f, r0 = 0.0f, r1 = 0.0f;
#pragma unroll
    for (int i = 0; i < PER_WAVE; ++i) {
        const float f = ml[i].x == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(ml[i].x - M);
        l = fmaf(f, ml[i].y, l);
        r0 = fmaf(f, ov[i].x, r0);
        r1 = fmaf(f, ov[i].y, r1);
    }
    sm.mo[wave][lane] = make_float2(r0, r1);
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
            const float f = m == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m - Mt);
            lt = fmaf(f, sm.wml[w][0][1], lt);
            const float2 o = sm.mo[w][lane];
            a0 = fmaf(f, o.x, a0);
            a1 = fmaf(f, o.y, a1);
        }
        const float inv = 1.0f / lt;
        ll_store(reinterpret_cast<uint64_t*>(a.attn_ll) + (hq * DL_D) / 2 + lane, ll_pack16x2(a0 * inv, a1 * inv, e_attn));
    }
}

// ------------------------------------------------------------- the kernel ----

// The arguments of the 256 / NB sequences one launch runs (block b serves sequence b / NB).
template <int NSEQ>
struct DlArgsSet {
    DlArgs s[NSEQ];
};

template <class S, bool TRACE>
__global__ __launch_bounds__(DL_THREADS) void decode_layers_kernel(const DlArgsSet<S::NSEQ> as) {
    __shared__ __align__(16) DlShared<S> sm;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // this block's sequence and its place among that sequence's NB blocks
    const int lb = blockIdx.x % S::NB;
    const DlArgs& a = as.s[blockIdx.x / S::NB];
    // The launch counter (written by block 0 of the previous launch) and the
    // position (written by the token-store kernel) are read with agent-scope
    // atomic loads: a plain scalar load can return a stale copy on another XCD,
    // and a block with a stale counter computes every epoch for the wrong launch.
    const uint32_t seq = __builtin_amdgcn_readfirstlane(
        __hip_atomic_load(a.ctl, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
    const int pos = __builtin_amdgcn_readfirstlane(
        __hip_atomic_load(const_cast<int32_t*>(a.pos_ptr), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
    const int L = pos + 1 < (int)a.s_cap ? pos + 1 : (int)a.s_cap;
    // RoPE at `pos` for the rotation pair (lane, lane + 64) of a head: the same in every layer of the launch
    float rope_cs = 1.0f, rope_sn = 0.0f;
    if (a.theta > 0.0f) {
        const int lane = threadIdx.x & 63;
        const float inv_freq = exp2f(-(2.0f * (float)lane / (float)DL_D) * log2f(a.theta));
        sincosf((float)pos * inv_freq, &rope_sn, &rope_cs);
    }
    const int kvh = lb % 8, bs = lb / 8;

    // The layer table is copied into LDS once.  Read from memory, each layer's
    // pointers would be a scalar-cache miss per launch, and a scalar load
    // shares its wait counter with LDS: the LDS waits after it would stall for
    // the miss (microseconds under load) wherever a phase first needs a pointer.
    __shared__ uint64_t tbl[DL_MAX_LAYERS * DL_LAYER_PTRS];
    for (uint32_t i = threadIdx.x; i < a.n_layers * DL_LAYER_PTRS; i += DL_THREADS) tbl[i] = a.layers[i];
    __syncthreads();
    auto layer_ptr = [&](uint32_t layer, int field) -> uint64_t {
        const uint64_t v = tbl[layer * DL_LAYER_PTRS + field];
        const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
        const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
        return (uint64_t)hi << 32 | lo;
    };
    auto make_rows = [&](uint32_t layer, int f0, int f1, uint32_t n_rows) {
        DlRows r;
        r.w0 = dl_gptr<const uint8_t>(layer_ptr(layer, f0));
        r.w1 = dl_gptr<const uint8_t>(layer_ptr(layer, f1));
        r.n_rows = r.n_rows4 = n_rows;
        r.w6 = nullptr;
        r.skip = 0;
        return r;
    };
    // q | k | v rows, contiguous (q | k only when v is Q6_K: the DL_FMT_Q4_TAIL6 phase sets n_rows4 and w6)
    auto qkv_rows = [&](uint32_t layer) { return make_rows(layer, DL_WQ, DL_WQ, S::QKV_ROWS); };
    auto o_rows = [&](uint32_t layer) { return make_rows(layer, DL_WO, DL_WO, S::HID); };
    auto gu_rows = [&](uint32_t layer) { return make_rows(layer, DL_WGATE, DL_WUP, S::MLP); };
    auto down_rows = [&](uint32_t layer) { return make_rows(layer, DL_WDOWN, DL_WDOWN, S::HID); };
    // Up to DL_WAVES * DL_ATT_POS positions, block bs = 0 of each kv head covers them all (32 per wave) and
    // writes the normalised output itself: no partials, no merge phase and no hand-off into it.  Longer, the
    // kv head's positions are spread over its S::ATT_SLOTS blocks and merged per q head.
    const bool att_direct = L <= DL_WAVES * DL_ATT_POS;
    const bool att_block = !att_direct || bs == 0;
    const int span = att_direct ? DL_ATT_POS : dl_att_span<S::ATT_SLOTS>(L);
    const int att_p0 = att_direct ? wave * DL_ATT_POS : (bs * DL_WAVES + wave) * span;
    const int att_rows = att_block ? dl_att_rows(L, att_p0, span) : 0;
    // phases with fewer units than waves spread them over the blocks
    constexpr int NB = S::NB;
    constexpr bool qkv_sp = S::QKV_ROWS / DlUnit<S::HSB, 1>::RPW < S::NW;
    constexpr bool o_sp = S::HID / DlUnit<S::QSB, 1>::RPW < S::NW;
    constexpr bool gu_sp = S::MLP / DlUnit<S::HSB, 2>::RPW < S::NW;
    constexpr bool dn_sp = S::HID / DlUnit<S::MSB, 1>::RPW < S::NW;
    // spread Q|K|V units also fit the blocks other than the direct attention's 8
    constexpr bool qkv_skip_ok =
        DL_QKV_SKIP && qkv_sp && S::QKV_ROWS / DlUnit<S::HSB, 1>::RPW <= (NB - 8) * DL_WAVES;
    static_assert((S::QKV_ROWS / DlUnit<S::HSB, 1>::RPW + S::NW - 1) / S::NW <= S::qkv_u &&
                      (S::HID / DlUnit<S::QSB, 1>::RPW + S::NW - 1) / S::NW <= S::o_u &&
                      (S::MLP / DlUnit<S::HSB, 2>::RPW + S::NW - 1) / S::NW <= S::gu_u &&
                      (S::HID / DlUnit<S::MSB, 1>::RPW + S::NW - 1) / S::NW <= S::dn_u,
                  "units per wave cover every unit");

    auto issue_bank = [&](uint32_t layer, DlAttnBank& bk) {
        dl_attn_issue_k(bk, dl_gptr<const uint16_t>(layer_ptr(layer, DL_K_CACHE)), kvh, att_p0, att_rows);
        dl_attn_issue_v(bk, dl_gptr<const uint16_t>(layer_ptr(layer, DL_V_CACHE)), kvh, att_p0, att_rows);
    };

    // A phase's first units are issued when the phase begins, after the phase
    // before has computed: a CU serves its waves' loads roughly in issue order,
    // so loads for a later phase issued any earlier would delay the current
    // phase's data in other waves (measured for gate|up, down and the next
    // layer's Q|K|V; only o_proj's units go early, see DL_O_EARLY).
    DlUnit<S::HSB, 1> uq[S::qkv_u];
    DlAttnBank bk;
    for (uint32_t layer = 0; layer < a.n_layers; ++layer) {
        const bool first = layer == 0, last = layer + 1 == a.n_layers;
        const uint32_t lsite = layer << 8;  // status code of a wait that gives up: layer and phase
        const uint32_t e_qkv = dl_epoch(seq, layer, DL_E_QKV), e_part = dl_epoch(seq, layer, DL_E_PART);
        const uint32_t e_attn = dl_epoch(seq, layer, DL_E_ATTN), e_ho = dl_epoch(seq, layer, DL_E_H_O);
        const uint32_t e_act = dl_epoch(seq, layer, DL_E_ACT), e_hd = dl_epoch(seq, layer, DL_E_H_DOWN);
        const uint32_t e_hprev = first ? 0u : dl_epoch(seq, layer - 1, DL_E_H_DOWN);
        const uint32_t wtypes = (uint32_t)layer_ptr(layer, DL_WTYPES);  // wave-uniform
        DlOut out;
        out.hold.kind = -1;
        // phase timeline slots of this block (the traced instantiation only)
        auto trp = [&](int phase) -> uint64_t* { return TRACE ? dl_trace_at(a, layer, phase) : nullptr; };
        out.tr = trp(0);
        dl_stamp(out.tr, DL_TR_BEGIN);
        // ---- Q|K|V: RMSNorm(h) . [Wq; Wk; Wv]^T.  The attention K/V rows depend
        // on nothing computed in this launch: they are issued with the Q|K|V
        // weights, before h is awaited, and stream during that hand-off.  A Q6_K
        // v: the q and k rows are Q4_K units and the v rows the Q6_K units that
        // follow them in the same unit numbering (each wave's last slot).
        out.ll32 = a.qkv_ll;
        out.e_out = e_qkv;
        const bool v6 = wtypes & DL_WT_V_Q6;
        DlRows qrows = qkv_rows(layer);
        // With the attention on one block per kv head (blocks 0..7), those blocks stream their kv head's whole
        // K/V rows during this phase: spread Q|K|V units go to the other blocks, which otherwise finished the
        // phase 0.8-1.4 us before them (traced at the 0.6B shape, KV 192)
        if constexpr (qkv_skip_ok) {
            if (att_direct) qrows.skip = 8;
        }
        if (v6) {
            qrows.n_rows4 = S::QD + S::KVD;
            qrows.w6 = dl_gptr<const uint8_t>(layer_ptr(layer, DL_WV));
            dl_issue_pre<S::HSB, 1, S::qkv_u, S::qkv_p, qkv_sp, NB, DL_FMT_Q4_TAIL6>(uq, qrows);
        } else {
            dl_issue_pre<S::HSB, 1, S::qkv_u, S::qkv_p, qkv_sp, NB, DL_FMT_Q4>(uq, qrows);
        }
        issue_bank(layer, bk);
        auto qkv_phase = [&](auto fmt) {
            dl_gemv_phase<S::HSB, 1, S::qkv_u, S::qkv_r, S::qkv_p, DL_EPI_STORE, true, qkv_sp, decltype(fmt)::value>(
                sm, uq, qrows, first ? DL_SRC_PLAIN : DL_SRC_LL32,
                first ? static_cast<const void*>(a.h) : static_cast<const void*>(a.h_ll), e_hprev,
                dl_gptr<const float>(layer_ptr(layer, DL_IN_NORM)), a.eps, out, a.status, lsite | DL_W_QKV);
        };
        if (v6)
            qkv_phase(std::integral_constant<int, DL_FMT_Q4_TAIL6>());
        else
            qkv_phase(std::integral_constant<int, DL_FMT_Q4>());
        dl_stamp(out.tr, DL_TR_END);
        // ---- attention split
        constexpr int o_early = DL_O_EARLY < S::o_r ? DL_O_EARLY : S::o_r;
        constexpr int o_pre = o_early > 0 ? o_early : S::o_p;
        DlUnit<S::QSB, 1> uo[S::o_u];
        {
            uint64_t* tr = trp(1);
            dl_stamp(tr, DL_TR_BEGIN);
            // only the fields the attention phase reads (each is two scalar registers)
            uint64_t lp[DL_LAYER_PTRS];
#pragma unroll
            for (int i = 0; i < DL_LAYER_PTRS; ++i) lp[i] = layer_ptr(layer, i);
            if (att_block) {
                dl_attn_phase<S>(bk, sm.at, a, lp, kvh, bs, att_p0, att_rows, att_direct, pos, rope_cs, rope_sn,
                                 e_qkv, att_direct ? e_attn : e_part, lsite, tr, [&] {
                                     if constexpr (o_early > 0)
                                         dl_issue_pre<S::QSB, 1, S::o_u, o_early, o_sp, NB>(uo, o_rows(layer));
                                 });
            } else if constexpr (o_early > 0) {
                dl_issue_pre<S::QSB, 1, S::o_u, o_early, o_sp, NB>(uo, o_rows(layer));
            }
            dl_stamp(tr, DL_TR_END);
        }
        // ---- attention merge (blocks 0..NH-1, one q head each)
        if (!att_direct && lb < S::NH) {
            uint64_t* tr = trp(2);
            dl_stamp(tr, DL_TR_BEGIN);
            dl_merge_phase<S>(sm.at, a, lb, e_part, e_attn, lsite, tr);
            dl_stamp(tr, DL_TR_END);
        }
        // ---- o_proj + residual
        out.tr = trp(3);
        dl_stamp(out.tr, DL_TR_BEGIN);
        if constexpr (o_early == 0) dl_issue_pre<S::QSB, 1, S::o_u, S::o_p, o_sp, NB>(uo, o_rows(layer));
        out.ll32 = a.h_ll;
        out.plain = nullptr;
        out.hold.kind = first ? DL_SRC_PLAIN : DL_SRC_LL32;
        out.hold.src = first ? static_cast<const void*>(a.h) : static_cast<const void*>(a.h_ll);
        out.hold.e = e_hprev;
        out.e_out = e_ho;
        dl_gemv_phase<S::QSB, 1, S::o_u, S::o_r, o_pre, DL_EPI_RESID, false, o_sp>(
            sm, uo, o_rows(layer), DL_SRC_LL16, a.attn_ll, e_attn, nullptr, a.eps, out, a.status, lsite | DL_W_O);
        dl_stamp(out.tr, DL_TR_END);
        // ---- RMSNorm + gate|up + SwiGLU
        out.tr = trp(4);
        dl_stamp(out.tr, DL_TR_BEGIN);
        DlUnit<S::HSB, 2> ug[S::gu_u];
        dl_issue_pre<S::HSB, 2, S::gu_u, S::gu_p, gu_sp, NB>(ug, gu_rows(layer));
        out.ll16 = a.act_ll;
        out.e_out = e_act;
        dl_gemv_phase<S::HSB, 2, S::gu_u, S::gu_r, S::gu_p, DL_EPI_SWIGLU, true, gu_sp>(
            sm, ug, gu_rows(layer), DL_SRC_LL32, a.h_ll, e_ho, dl_gptr<const float>(layer_ptr(layer, DL_POST_NORM)),
            a.eps, out, a.status, lsite | DL_W_GU);
        dl_stamp(out.tr, DL_TR_END);
        // ---- down + residual (the last layer writes the caller's h); Q4_K or Q6_K rows
        out.tr = trp(5);
        dl_stamp(out.tr, DL_TR_BEGIN);
        out.ll32 = a.h_ll;
        out.plain = last ? a.h : nullptr;
        out.hold.kind = DL_SRC_LL32;
        out.hold.src = a.h_ll;
        out.hold.e = e_ho;
        out.e_out = e_hd;
        auto down_phase = [&](auto fmt) {
            constexpr int FMT = decltype(fmt)::value;
            DlUnit<S::MSB, 1> ud[S::dn_u];
            dl_issue_pre<S::MSB, 1, S::dn_u, S::dn_p, dn_sp, NB, FMT>(ud, down_rows(layer));
            dl_gemv_phase<S::MSB, 1, S::dn_u, S::dn_r, S::dn_p, DL_EPI_RESID, false, dn_sp, FMT>(
                sm, ud, down_rows(layer), DL_SRC_LL16, a.act_ll, e_act, nullptr, a.eps, out, a.status,
                lsite | DL_W_DOWN);
        };
        if (wtypes & DL_WT_DOWN_Q6)
            down_phase(std::integral_constant<int, DL_FMT_Q6>());
        else
            down_phase(std::integral_constant<int, DL_FMT_Q4>());
        dl_stamp(out.tr, DL_TR_END);
    }
    // Every block of the sequence has read the launch counter before its block 0
    // can get here: its last phase consumed every block's output.
    if (lb == 0 && threadIdx.x == 0)
        __hip_atomic_store(a.ctl, seq + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

static size_t dl_align(size_t v) { return (v + 255) & ~(size_t)255; }

// ------------------------------------------- allocation-free entry point ----

// Workspace of t2h_qwen3_decode_layers_noalloc: one per GPU, held until the
// process ends, zero at load (a zero launch counter and no valid epoch).  Large
// enough for every built shape's layout (8B: 1.16 MiB, 0.6B: 0.6 MiB).
constexpr size_t DL_SCRATCH_BYTES = (size_t)3 << 19;  // 1.5 MiB
static __device__ __align__(256) uint8_t scratch[DL_SCRATCH_BYTES];
constexpr int DL_MAX_DEVICES = 64;
static std::atomic<void*> dl_scratch_ptr[DL_MAX_DEVICES];
static std::mutex dl_scratch_mu;

// The device address of the current GPU's copy of `scratch`, looked up on the
// first call on that GPU (hipGetSymbolAddress, with the GPU current) and kept:
// in host code the array's name is not a device address.
static int dl_scratch(void** out) {
    int dev = 0;
    const hipError_t ge = hipGetDevice(&dev);
    if (ge != hipSuccess) return T2H_ERR_HIP_BASE + (int)ge;
    if (dev < 0 || dev >= DL_MAX_DEVICES) return T2H_ERR_UNSUPPORTED;
    void* p = dl_scratch_ptr[dev].load(std::memory_order_acquire);
    if (p == nullptr) {
        std::lock_guard<std::mutex> lock(dl_scratch_mu);
        p = dl_scratch_ptr[dev].load(std::memory_order_relaxed);
        if (p == nullptr) {
            const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
            if (e != hipSuccess) return T2H_ERR_HIP_BASE + (int)e;
            if (p == nullptr) return T2H_ERR_NULL;
            dl_scratch_ptr[dev].store(p, std::memory_order_release);
        }
    }
    *out = p;
    return T2H_OK;
}

struct DlLayout {
    size_t ctl, qkv, attn, act, h, part, total;
};

// Workspace: launch counter, then the epoch-tagged vectors.
template <class S>
static DlLayout dl_layout() {
    DlLayout l;
    size_t off = 0;
    l.ctl = off;
    off += 256;
    l.qkv = off;
    off += dl_align((size_t)S::QKV_ROWS * 8);
    l.attn = off;
    off += dl_align((size_t)S::QD * 4);
    l.act = off;
    off += dl_align((size_t)S::MLP * 4);
    l.h = off;
    off += dl_align((size_t)S::HID * 8);
    l.part = off;
    off += dl_align((size_t)S::NK * DL_ATT_SLOTS * S::GROUP * (2 + DL_D) * 8);
    l.total = off;
    return l;
}

// Cached residency check per shape: 1 = 256 blocks fit on the device at once.
template <class S>
static bool dl_grid_fits() {
    static int fits = -1;
    if (fits >= 0) return fits == 1;
    int dev = 0, cus = 0, per_cu = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, decode_layers_kernel<S, false>, DL_THREADS, 0) !=
            hipSuccess) {
        fits = 0;
        return false;
    }
    fits = (cus * per_cu >= DL_BLOCKS) ? 1 : 0;
    return fits == 1;
}

template <class S>
static bool dl_is(uint32_t hidden, uint32_t mlp, uint32_t nh, uint32_t nk, uint32_t d) {
    return hidden == (uint32_t)S::HID && mlp == (uint32_t)S::MLP && nh == (uint32_t)S::NH && nk == (uint32_t)S::NK &&
           d == (uint32_t)DL_D;
}

// One sequence's arguments over its workspace (laid out by dl_layout).
template <class S>
static int dl_args(DlArgs& a, const uint64_t* layer_table, uint32_t n_layers, uint32_t s_cap, float* h,
                   const int32_t* cache_position, float eps, float theta, void* workspace, size_t workspace_bytes,
                   uint32_t* status, uint64_t* trace) {
    const DlLayout l = dl_layout<S>();
    if (workspace_bytes < l.total) return T2H_ERR_WORKSPACE;
    if (reinterpret_cast<uintptr_t>(workspace) % 256 != 0) return T2H_ERR_ALIGN;
    uint8_t* ws = reinterpret_cast<uint8_t*>(workspace);
    a.layers = layer_table;
    a.n_layers = n_layers;
    a.h = h;
    a.pos_ptr = cache_position;
    a.s_cap = s_cap;
    a.eps = eps;
    a.theta = theta;
    a.ctl = reinterpret_cast<uint32_t*>(ws + l.ctl);
    a.qkv_ll = reinterpret_cast<uint64_t*>(ws + l.qkv);
    a.attn_ll = reinterpret_cast<uint32_t*>(ws + l.attn);
    a.act_ll = reinterpret_cast<uint32_t*>(ws + l.act);
    a.h_ll = reinterpret_cast<uint64_t*>(ws + l.h);
    a.part_ll = reinterpret_cast<uint64_t*>(ws + l.part);
    a.status = status;
    a.trace = trace;
    return T2H_OK;
}

template <class S>
static int dl_launch(const uint64_t* layer_table, uint32_t n_layers, uint32_t s_cap, float* h,
                     const int32_t* cache_position, float eps, float theta, void* workspace, size_t workspace_bytes,
                     uint32_t* status, uint64_t* trace, void* stream) {
    static_assert(S::NSEQ == 1, "one sequence");
    DlArgsSet<1> as;
    const int rc = dl_args<S>(as.s[0], layer_table, n_layers, s_cap, h, cache_position, eps, theta, workspace,
                              workspace_bytes, status, trace);
    if (rc != T2H_OK) return rc;
    if (!dl_grid_fits<S>()) return T2H_ERR_UNSUPPORTED;
    if (trace == nullptr)
        hipLaunchKernelGGL((decode_layers_kernel<S, false>), dim3(DL_BLOCKS), dim3(DL_THREADS), 0,
                           reinterpret_cast<hipStream_t>(stream), as);
    else
        hipLaunchKernelGGL((decode_layers_kernel<S, true>), dim3(DL_BLOCKS), dim3(DL_THREADS), 0,
                           reinterpret_cast<hipStream_t>(stream), as);
    T2H_LAUNCH_CHECK();
    return T2H_OK;
}

// S::NSEQ sequences side by side, sequence i on blocks [i NB, (i + 1) NB).
// trace: one timeline buffer for the launch (t2h_qwen3_decode_layers_trace_bytes), indexed by the grid's block,
// so sequence i's stamps are blocks [i NB, (i + 1) NB); null for the untraced instantiation.
template <class S>
static int dl_launch_seqs(const uint64_t* const* layer_tables, uint32_t n_layers, uint32_t s_cap, float* const* hs,
                          const int32_t* const* cache_positions, float eps, float theta, void* const* workspaces,
                          size_t workspace_bytes, uint32_t* const* statuses, uint64_t* trace, void* stream) {
    DlArgsSet<S::NSEQ> as;
    for (int i = 0; i < S::NSEQ; ++i) {
        if (!layer_tables[i] || !hs[i] || !cache_positions[i] || !workspaces[i] || !statuses[i]) return T2H_ERR_NULL;
        const int rc = dl_args<S>(as.s[i], layer_tables[i], n_layers, s_cap, hs[i], cache_positions[i], eps, theta,
                                  workspaces[i], workspace_bytes, statuses[i], trace);
        if (rc != T2H_OK) return rc;
        for (int j = 0; j < i; ++j)
            if (workspaces[j] == workspaces[i]) return T2H_ERR_ARG;  // each sequence needs its own workspace
    }
    if (!dl_grid_fits<S>()) return T2H_ERR_UNSUPPORTED;
    if (trace == nullptr)
        hipLaunchKernelGGL((decode_layers_kernel<S, false>), dim3(DL_BLOCKS), dim3(DL_THREADS), 0,
                           reinterpret_cast<hipStream_t>(stream), as);
    else
        hipLaunchKernelGGL((decode_layers_kernel<S, true>), dim3(DL_BLOCKS), dim3(DL_THREADS), 0,
                           reinterpret_cast<hipStream_t>(stream), as);
    T2H_LAUNCH_CHECK();
    return T2H_OK;
}

}  // namespace t2h
using namespace t2h;


extern "C" size_t t2h_qwen3_decode_layers_workspace_bytes(uint32_t hidden, uint32_t mlp, uint32_t nh, uint32_t nk,
                                                         uint32_t d) {
    if (dl_is<DlQwen3_8B>(hidden, mlp, nh, nk, d)) return dl_layout<DlQwen3_8B>().total;
    if (dl_is<DlQwen3_0_6B>(hidden, mlp, nh, nk, d)) return dl_layout<DlQwen3_0_6B>().total;
    if (dl_is<DlQwen3_1_7B>(hidden, mlp, nh, nk, d)) return dl_layout<DlQwen3_1_7B>().total;
    return 0;
}

static int dl_entry(const uint64_t* layer_table, uint32_t n_layers, uint32_t hidden, uint32_t mlp, uint32_t nh,
                    uint32_t nk, uint32_t d, uint32_t s_cap, float* h, const int32_t* cache_position, float eps,
                    float theta, void* workspace, size_t workspace_bytes, uint32_t* status, uint64_t* trace,
                    void* stream) {
    if (!layer_table || !h || !cache_position || !workspace || !status) return T2H_ERR_NULL;
    const bool is8b = dl_is<DlQwen3_8B>(hidden, mlp, nh, nk, d), is1_7b = dl_is<DlQwen3_1_7B>(hidden, mlp, nh, nk, d);
    if (!is8b && !is1_7b && !dl_is<DlQwen3_0_6B>(hidden, mlp, nh, nk, d)) return T2H_ERR_UNSUPPORTED;
    if (n_layers == 0) return T2H_OK;
    if (n_layers > DL_MAX_LAYERS) return T2H_ERR_UNSUPPORTED;
    if (s_cap == 0) return T2H_ERR_SHAPE;
    if ((size_t)(s_cap + DL_ATT_SLOTS * DL_WAVES - 1) / (DL_ATT_SLOTS * DL_WAVES) > DL_ATT_POS)
        return T2H_ERR_UNSUPPORTED;  // more than 32 positions per wave
    if (is8b)
        return dl_launch<DlQwen3_8B>(layer_table, n_layers, s_cap, h, cache_position, eps, theta, workspace,
                                     workspace_bytes, status, trace, stream);
    if (is1_7b)
        return dl_launch<DlQwen3_1_7B>(layer_table, n_layers, s_cap, h, cache_position, eps, theta, workspace,
                                       workspace_bytes, status, trace, stream);
    return dl_launch<DlQwen3_0_6B>(layer_table, n_layers, s_cap, h, cache_position, eps, theta, workspace,
                                   workspace_bytes, status, trace, stream);
}

extern "C" int t2h_qwen3_decode_layers(const uint64_t* layer_table, uint32_t n_layers, uint32_t hidden, uint32_t mlp,
                                       uint32_t nh, uint32_t nk, uint32_t d, uint32_t s_cap, float* h,
                                       const int32_t* cache_position, float eps, float theta, void* workspace,
                                       size_t workspace_bytes, uint32_t* status, void* stream) {
    return dl_entry(layer_table, n_layers, hidden, mlp, nh, nk, d, s_cap, h, cache_position, eps, theta, workspace,
                    workspace_bytes, status, nullptr, stream);
}

extern "C" int t2h_qwen3_decode_layers_noalloc(const uint64_t* layer_table, uint32_t n_layers, uint32_t hidden,
                                               uint32_t mlp, uint32_t nh, uint32_t nk, uint32_t d, uint32_t s_cap,
                                               float* h, const int32_t* cache_position, float eps, float theta,
                                               uint32_t* status, void* stream) {
    const size_t need = t2h_qwen3_decode_layers_workspace_bytes(hidden, mlp, nh, nk, d);
    if (need == 0) return T2H_ERR_UNSUPPORTED;
    if (need > DL_SCRATCH_BYTES) return T2H_ERR_WORKSPACE;  // a shape whose workspace the array cannot hold
    void* ws = nullptr;
    const int rc = dl_scratch(&ws);
    if (rc != T2H_OK) return rc;
    return dl_entry(layer_table, n_layers, hidden, mlp, nh, nk, d, s_cap, h, cache_position, eps, theta, ws,
                    DL_SCRATCH_BYTES, status, nullptr, stream);
}

extern "C" size_t t2h_qwen3_decode_layers_trace_bytes(uint32_t n_layers) {
    return (size_t)n_layers * DL_TR_PHASES * DL_BLOCKS * DL_TR_SLOTS * sizeof(uint64_t);
}

extern "C" int t2h_qwen3_decode_layers_traced(const uint64_t* layer_table, uint32_t n_layers, uint32_t hidden,
                                              uint32_t mlp, uint32_t nh, uint32_t nk, uint32_t d, uint32_t s_cap,
                                              float* h, const int32_t* cache_position, float eps, float theta,
                                              void* workspace, size_t workspace_bytes, uint32_t* status,
                                              uint64_t* trace, size_t trace_bytes, void* stream) {
    if (!trace) return T2H_ERR_NULL;
    if (trace_bytes < t2h_qwen3_decode_layers_trace_bytes(n_layers)) return T2H_ERR_WORKSPACE;
    if (reinterpret_cast<uintptr_t>(trace) % 8 != 0) return T2H_ERR_ALIGN;
    return dl_entry(layer_table, n_layers, hidden, mlp, nh, nk, d, s_cap, h, cache_position, eps, theta, workspace,
                    workspace_bytes, status, trace, stream);
}

static int dl_entry_seqs(uint32_t n_seq, const uint64_t* const* layer_tables, uint32_t n_layers, uint32_t hidden,
                         uint32_t mlp, uint32_t nh, uint32_t nk, uint32_t d, uint32_t s_cap, float* const* hs,
                         const int32_t* const* cache_positions, float eps, float theta, void* const* workspaces,
                         size_t workspace_bytes, uint32_t* const* statuses, uint64_t* trace, void* stream) {
    if (!layer_tables || !hs || !cache_positions || !workspaces || !statuses) return T2H_ERR_NULL;
    if (n_seq == 1)
        return dl_entry(layer_tables[0], n_layers, hidden, mlp, nh, nk, d, s_cap, hs[0], cache_positions[0], eps,
                        theta, workspaces[0], workspace_bytes, statuses[0], trace, stream);
    if (n_seq != (uint32_t)DlQwen3_0_6B_x4::NSEQ || !dl_is<DlQwen3_0_6B_x4>(hidden, mlp, nh, nk, d))
        return T2H_ERR_UNSUPPORTED;
    if (n_layers == 0) return T2H_OK;
    if (n_layers > DL_MAX_LAYERS) return T2H_ERR_UNSUPPORTED;
    if (s_cap == 0) return T2H_ERR_SHAPE;
    constexpr uint32_t waves = DlQwen3_0_6B_x4::ATT_SLOTS * DL_WAVES;
    if ((size_t)(s_cap + waves - 1) / waves > DL_ATT_POS) return T2H_ERR_UNSUPPORTED;  // over 32 positions a wave
    return dl_launch_seqs<DlQwen3_0_6B_x4>(layer_tables, n_layers, s_cap, hs, cache_positions, eps, theta, workspaces,
                                            workspace_bytes, statuses, trace, stream);
}

extern "C" int t2h_qwen3_decode_layers_seqs(uint32_t n_seq, const uint64_t* const* layer_tables, uint32_t n_layers,
                                            uint32_t hidden, uint32_t mlp, uint32_t nh, uint32_t nk, uint32_t d,
                                            uint32_t s_cap, float* const* hs, const int32_t* const* cache_positions,
                                            float eps, float theta, void* const* workspaces, size_t workspace_bytes,
                                            uint32_t* const* statuses, void* stream) {
    return dl_entry_seqs(n_seq, layer_tables, n_layers, hidden, mlp, nh, nk, d, s_cap, hs, cache_positions, eps, theta,
                         workspaces, workspace_bytes, statuses, nullptr, stream);
}

extern "C" int t2h_qwen3_decode_layers_seqs_traced(uint32_t n_seq, const uint64_t* const* layer_tables,
                                                   uint32_t n_layers, uint32_t hidden, uint32_t mlp, uint32_t nh,
                                                   uint32_t nk, uint32_t d, uint32_t s_cap, float* const* hs,
                                                   const int32_t* const* cache_positions, float eps, float theta,
                                                   void* const* workspaces, size_t workspace_bytes,
                                                   uint32_t* const* statuses, uint64_t* trace, size_t trace_bytes,
                                                   void* stream) {
    if (!trace) return T2H_ERR_NULL;
    if (trace_bytes < t2h_qwen3_decode_layers_trace_bytes(n_layers)) return T2H_ERR_WORKSPACE;
    if (reinterpret_cast<uintptr_t>(trace) % 8 != 0) return T2H_ERR_ALIGN;
    return dl_entry_seqs(n_seq, layer_tables, n_layers, hidden, mlp, nh, nk, d, s_cap, hs, cache_positions, eps, theta,
                         workspaces, workspace_bytes, statuses, trace, stream);
}
