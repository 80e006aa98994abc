// Flash attention for prefill / encoders on the gfx950 matrix cores.
//
// Replaces the reference's prefill attention shaders:
//   LLAMA_FLASH_ATTN_F32_F16_F16 (+ FA_MASK_OPT_F16)  token-major q/k/v, additive mask
//       src/models/optimized_qwen3/shaders/llama_flash_attn_f32_f16_f16.py:35-175
//   SDPA_CAUSAL_F32      head-major, causal      src/models/quantized_qwen3/shaders/sdpa_causal_f32.py:22-142
//   SDPA_MASKED_F32      head-major, additive mask (the Qwen3-ASR audio encoder)
//       src/models/optimized_qwen3_asr/shaders/sdpa_masked_f32.py
// Every tensor is addressed through (batch, token, head) strides with the
// head dimension contiguous, so both layouts run through one kernel.
//
// Math: out[b,t,h] = softmax(q.k^T * scale + mask) v over the keys a query may
// see (causal: key <= t + causal_offset; segments: the keys of the query's own
// segment), GQA kv head = h / (NH / NK); fp32 scores, running max and sum,
// bf16 P, fp32 output accumulation.
//
// Segments.  The Qwen3-ASR encoder attends within windows: its additive mask is
// 0 on diagonal blocks [cu[i], cu[i+1]) and -FLT_MAX elsewhere
// (src/models/quantized_qwen3_asr/pytorch_modules.py:95-114).  Given the window
// bounds cu[] instead of the mask, every query's keys are one interval
// [lo, hi): each block takes queries of one segment, visits its keys in tiles
// from the segment's first key on, and masks only the last, partial tile.
//
// Work mapping.  A block of 4 waves takes 128 queries of one (batch, head);
// wave w owns 32 of them.  Keys stream through LDS 64 at a time, double
// buffered: the next tile's K rows and V columns are in flight to registers
// while the matrix cores work on the current one.
//   * S^T = K . Q^T on v_mfma_f32_32x32x16_bf16: K rows come from LDS, the
//     wave's Q^T columns stay in registers for the whole pass.  In the
//     accumulator layout a lane then holds one query's scores for 16 keys, so
//     the row max and sum are in-lane plus one exchange between the two
//     half-waves (the other 16 keys of each 32).
//   * O^T += V^T . P^T: the accumulator registers of S^T, scaled, exponentiated
//     and packed to bf16, are already the B operand of the second product when
//     its 16 k-slots are assigned to the keys each lane holds; the A operand
//     reads V^T from LDS with the same key order.  V goes into LDS as it is in
//     memory, [key][dim], and the transposing LDS read (ds_read_b64_tr_b16)
//     hands each lane one dim of 4 consecutive keys.
//   * Tile loads: every full tile's K and V rows are at fixed per-thread
//     offsets from a wave-uniform tile base; only the last, partial tile clamps
//     its keys to the sequence.
// Operand layout of v_mfma_f32_32x32x16_bf16: lane l supplies row (l % 32) of
// A and column (l % 32) of B, 8 consecutive k each, k = 8 (l / 32) + j; its 16
// results are C[8(i/4) + 4(l/32) + i%4][l % 32].
#include "common.h"

namespace t2h {

typedef __bf16 fa_bf16x8_t __attribute__((ext_vector_type(8)));
typedef float fa_f32x16_t __attribute__((ext_vector_type(16)));

constexpr int FA_WAVES = 4;
constexpr int FA_THREADS = FA_WAVES * 64;
constexpr int FA_BM = 32 * FA_WAVES;  // queries per block
constexpr int FA_BN = 64;             // keys per tile

constexpr float FA_LOG2E = 1.4426950408889634f;
constexpr float FA_RESCALE = 8.0f;    // log2 headroom of the lazily updated running max

struct FaArgs {
    const uint16_t* q;  // bf16
    const uint16_t* k;
    const uint16_t* v;
    uint16_t* out;
    const float* mask;  // additive, natural-log units; null = none
    const int32_t* cu;  // segment bounds [n_seg + 1] (SEG kernels)
    uint32_t n_seg;
    size_t q_sb, q_st, q_sh;
    size_t k_sb, k_st, k_sh;
    size_t v_sb, v_st, v_sh;
    size_t o_sb, o_st, o_sh;
    size_t m_sb, m_st;
    uint32_t nh;
    uint32_t group;  // q heads per kv head
    uint32_t batch;
    uint32_t t_len;
    uint32_t s_len;
    int32_t causal_offset;
    float scale_log2;  // softmax scale * log2(e)
    const uint8_t* tiles;  // MASK: class of each (query block, key tile) of the mask, or null
    size_t tiles_sb;       // batch stride of tiles (0: one mask for every batch)
    uint32_t n_tiles;      // key tiles per query block row of tiles
};

// Mask tile classes (the reference's FA_MASK_OPT_F16: all masked / all zero / mixed), per block of FA_BM
// queries x FA_BN keys.  A value at or below -FA_MASKED masks its key.
enum FaTile { FA_TILE_MIXED = 0, FA_TILE_MASKED = 1, FA_TILE_ZERO = 2 };
constexpr float FA_MASKED = 1.7014117e38f;  // FLT_MAX / 2

__device__ __forceinline__ fa_bf16x8_t as_bf16x8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    return __builtin_bit_cast(fa_bf16x8_t, make_uint4(a, b, c, d));
}

// Block -> (query block, batch, head).  Blocks go round-robin to the 8 XCDs; when the (batch, kv head) groups
// split evenly over them, each XCD takes whole groups one after another (a group's K/V rows then stay in that
// XCD's L2 while its blocks run), and within a group the query blocks with the most keys start first; else
// the longest query blocks start first over the whole grid.
__device__ __forceinline__ void fa_block(const FaArgs& a, int nqb, int& qb, int& b, int& h) {
    const int L = blockIdx.x;
    const int nk = (int)(a.nh / a.group);
    const int groups = (int)a.batch * nk;
    if (groups % 8 == 0) {
        const int x = L % 8, j = L / 8;
        const int per_grp = nqb * (int)a.group;  // blocks of one (batch, kv head) group
        const int grp = x + 8 * (j / per_grp);
        const int r = j % per_grp;
        qb = nqb - 1 - r / (int)a.group;
        b = grp / nk;
        h = (grp % nk) * (int)a.group + r % (int)a.group;
    } else {
        const int bh = (int)a.batch * (int)a.nh;
        qb = nqb - 1 - L / bh;
        b = (L % bh) / (int)a.nh;
        h = (L % bh) % (int)a.nh;
    }
}

// Segments: the query blocks of each segment start at its first token, so that no block holds queries of two
// segments (it would visit the keys of both, twice the tiles of its neighbours).  The table is extended to
// E = [0, cu[0], ..., cu[n_seg], t_len], each bound clamped to [0, t_len]; segment i of E is [E_i, E_i+1), the
// first and the last being the tokens outside the table, which see no keys.  Segment i owns the blocks
// [f(i), f(i + 1)) of a (batch, head), f(i) = floor(E_i / FA_BM) + i: at least ceil(len_i / FA_BM) of them
// (a spare one finds no queries and exits), so f(n_seg + 2) blocks cover every token.  f ascends with E, and a
// binary search finds a block's segment; a table that does not ascend gives wrong windows, never an access
// outside [0, t_len).
__device__ __forceinline__ int fa_ext_bound(const FaArgs& a, int i) {
    if (i <= 0) return 0;
    if (i >= (int)a.n_seg + 2) return (int)a.t_len;
    return min(max(a.cu[i - 1], 0), (int)a.t_len);
}

// Queries [q0, q_end) and keys [lo, hi) of virtual block vb of a (batch, head); false when it has no queries.
__device__ __forceinline__ bool fa_seg_block(const FaArgs& a, int vb, int& q0, int& q_end, int& lo, int& hi) {
    const int n = (int)a.n_seg;
    int l = 0, r = n + 2;  // f(l) <= vb < f(r)
    while (r - l > 1) {
        const int mid = (l + r) >> 1;
        if (fa_ext_bound(a, mid) / FA_BM + mid <= vb) l = mid;
        else r = mid;
    }
    const int s_lo = fa_ext_bound(a, l);
    const int s_hi = max(s_lo, fa_ext_bound(a, l + 1));
    q0 = (int)min((long long)s_lo + (long long)(vb - (s_lo / FA_BM + l)) * FA_BM, (long long)s_hi);
    q_end = min(q0 + FA_BM, s_hi);
    const bool in_table = l >= 1 && l <= n;
    lo = in_table ? s_lo : 0;
    hi = in_table ? s_hi : 0;
    return q0 < q_end;
}

// Keys [lo, hi) that query q may see, clamped to [0, s_len).
template <bool CAUSAL>
__device__ __forceinline__ int2 fa_key_range(const FaArgs& a, int q) {
    int lo = 0, hi = (int)a.s_len;
    if constexpr (CAUSAL) hi = min(hi, q + a.causal_offset + 1);
    return make_int2(lo, max(lo, hi));
}

template <int D, bool CAUSAL, bool MASK, bool SEG>
__global__ __launch_bounds__(FA_THREADS) __attribute__((amdgpu_waves_per_eu(MASK ? 1 : 2))) void fa_prefill_kernel(const FaArgs a) {
    constexpr int KROW = D + 8;                                // LDS K row length (bf16)
    // LDS V row length: 2 VROW = 64 (mod 256) bytes, so the 4 rows x 64 B that each half-wave of a
    // transposing read addresses fall on distinct banks (D + 16 measured 25 % bank conflicts)
    constexpr int VROW = D + 32;
    constexpr int DS = D / 16;                                 // k-steps of S^T
    constexpr int DB = D / 32;                                 // 32-dim blocks of O^T
    constexpr int CPR = D / 8;                                 // 16-B chunks per K or V row
    constexpr int KCH = FA_BN * CPR / FA_THREADS;              // chunks of each per thread
    static_assert(KCH >= 1 && FA_THREADS % CPR == 0, "tile too small for the block");
    __shared__ __align__(16) uint16_t ks[2][FA_BN * KROW];
    __shared__ __align__(16) uint16_t vs[2][FA_BN * VROW];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int half = lane >> 5;
    int qb, b, h;
    fa_block(a, SEG ? (int)(a.t_len / FA_BM) + (int)a.n_seg + 2 : ((int)a.t_len + FA_BM - 1) / FA_BM, qb, b, h);
    const int kvh = h / a.group;
    int q0, q_end = (int)a.t_len, seg_lo = 0, seg_hi = 0;
    if constexpr (SEG) {
        if (!fa_seg_block(a, qb, q0, q_end, seg_lo, seg_hi)) return;  // block-uniform, before any barrier
    } else {
        q0 = qb * FA_BM;
    }
    const int qi = q0 + 32 * wave + (lane & 31);  // this lane's query
    const bool q_valid = qi < q_end;
    const int qc = q_valid ? qi : q_end - 1;
    const int s_len = (int)a.s_len;

    // Key ranges only grow with the query index, so the block's queries see
    // [range(q0).lo, range(q_last).hi) and a wave's need no mask on the keys
    // between its last query's lo and its first query's hi.  A segment's
    // queries all see its keys, in tiles from its first key on.
    const int q_last = min(q0 + FA_BM, q_end) - 1;
    const int2 rq = SEG ? make_int2(seg_lo, seg_hi) : fa_key_range<CAUSAL>(a, qc);
    const int blk_lo = SEG ? seg_lo : fa_key_range<CAUSAL>(a, q0).x;
    const int blk_hi = SEG ? seg_hi : fa_key_range<CAUSAL>(a, q_last).y;
    const int key_base = SEG ? blk_lo : 0;  // key of tile 0
    int t_first = SEG ? 0 : blk_lo / FA_BN;
    int t_end = blk_hi > blk_lo ? (blk_hi - key_base + FA_BN - 1) / FA_BN : t_first;
    if constexpr (MASK) {
        // all-masked tiles at either end of the block's row of the mask are not visited at all
        if (a.tiles != nullptr) {
            const uint8_t* tr = a.tiles + (size_t)b * a.tiles_sb + (size_t)qb * a.n_tiles;
            while (t_first < t_end && tr[t_first] == FA_TILE_MASKED) ++t_first;
            while (t_end > t_first && tr[t_end - 1] == FA_TILE_MASKED) --t_end;
        }
    }
    const int wave_lo_max = __builtin_amdgcn_readlane(rq.x, 31);
    const int wave_hi_min = __builtin_amdgcn_readlane(rq.y, 0);

    // Q^T columns of this lane's query: dims 16 s + 8 half .. +7
    const uint16_t* qrow = a.q + (size_t)b * a.q_sb + (size_t)qc * a.q_st + (size_t)h * a.q_sh;
    fa_bf16x8_t qf[DS];
#pragma unroll
    for (int s = 0; s < DS; ++s) qf[s] = *reinterpret_cast<const fa_bf16x8_t*>(qrow + 16 * s + 8 * half);

    const uint16_t* kb_ptr = a.k + (size_t)b * a.k_sb + (size_t)kvh * a.k_sh;
    const uint16_t* vb_ptr = a.v + (size_t)b * a.v_sb + (size_t)kvh * a.v_sh;
    // chunk i of this thread: key row tid / CPR + i FA_THREADS / CPR of the tile, 8 dims at 8 (tid % CPR)
    const int ch_key = tid / CPR, ch_col = (tid % CPR) * 8;
    uint32_t koff[KCH], voff[KCH];  // element offsets from a full tile's first key row
#pragma unroll
    for (int i = 0; i < KCH; ++i) {
        koff[i] = (uint32_t)((ch_key + i * (FA_THREADS / CPR)) * a.k_st + ch_col);
        voff[i] = (uint32_t)((ch_key + i * (FA_THREADS / CPR)) * a.v_st + ch_col);
    }
    uint4 kreg[KCH], vreg[KCH];
    auto load_tile = [&](int t0) {
        if (t0 + FA_BN <= s_len) {
            const uint16_t* kt = kb_ptr + (size_t)t0 * a.k_st;  // wave-uniform
            const uint16_t* vt = vb_ptr + (size_t)t0 * a.v_st;
#pragma unroll
            for (int i = 0; i < KCH; ++i) {
                kreg[i] = load_u4(kt + koff[i]);
                // V rows are 8-B aligned: two 8-B halves
                const uint2 lo = *reinterpret_cast<const uint2*>(vt + voff[i]);
                const uint2 hi = *reinterpret_cast<const uint2*>(vt + voff[i] + 4);
                vreg[i] = make_uint4(lo.x, lo.y, hi.x, hi.y);
            }
        } else {
            // the sequence's last, partial tile: keys past the end read the last key again (never used)
#pragma unroll
            for (int i = 0; i < KCH; ++i) {
                const int key = min(t0 + ch_key + i * (FA_THREADS / CPR), s_len - 1);
                kreg[i] = load_u4(kb_ptr + (size_t)key * a.k_st + ch_col);
                const uint16_t* vr = vb_ptr + (size_t)key * a.v_st + ch_col;
                const uint2 lo = *reinterpret_cast<const uint2*>(vr);
                const uint2 hi = *reinterpret_cast<const uint2*>(vr + 4);
                vreg[i] = make_uint4(lo.x, lo.y, hi.x, hi.y);
            }
        }
    };
    auto store_tile = [&](int buf) {
#pragma unroll
        for (int i = 0; i < KCH; ++i) {
            const int key = ch_key + i * (FA_THREADS / CPR);
            *reinterpret_cast<uint4*>(&ks[buf][key * KROW + ch_col]) = kreg[i];
            *reinterpret_cast<uint4*>(&vs[buf][key * VROW + ch_col]) = vreg[i];
        }
    };
    // transposing V^T reads: lane 4 j + c of each 16-lane group addresses key row j of a 4-row block at dims
    // 4 c .. 4 c + 3 of the group's 16 dims, and receives one dim of the 4 keys
    const int n16 = lane & 15;
    const int v_lane = (4 * half + (n16 >> 2)) * VROW + 16 * ((lane >> 4) & 1) + 4 * (n16 & 3);

    fa_f32x16_t o[DB];
#pragma unroll
    for (int i = 0; i < DB; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) o[i][e] = 0.0f;
    float m_run = -INFINITY;  // log2-domain running max of this lane's query
    float l_part = 0.0f;      // this half-wave's share of the running sum

    if (t_end > t_first) {
        load_tile(key_base + t_first * FA_BN);
        store_tile(0);
    }
    // Every load issued so far (the q fragments included) has landed before the loop: the compiler's wait
    // analysis merges the state entering the loop with the state of its back edge, and with q possibly in
    // flight on entry it made each score MFMA wait for the next tile's loads in flight on the back edge.
    __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));  // vmcnt(0)
    __syncthreads();

    const float* mrow = nullptr;
    if constexpr (MASK) mrow = a.mask + (size_t)b * a.m_sb + (size_t)qc * a.m_st;
    // tile classes of this block's row of the mask (the range was already narrowed before the first load)
    const uint8_t* trow = nullptr;
    if constexpr (MASK) {
        if (a.tiles != nullptr) trow = a.tiles + (size_t)b * a.tiles_sb + (size_t)qb * a.n_tiles;
    }

    for (int t = t_first; t < t_end; ++t) {
        const int buf = (t - t_first) & 1;
        const int t0 = key_base + t * FA_BN;
        if (t + 1 < t_end) load_tile(t0 + FA_BN);
        const int cls = trow != nullptr ? (int)trow[t] : FA_TILE_MIXED;  // block-uniform
        if (cls != FA_TILE_MASKED) {

        // S^T for two 32-key blocks
        fa_f32x16_t s[2];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
            for (int e = 0; e < 16; ++e) s[kb][e] = 0.0f;
            const uint16_t* krow = &ks[buf][(32 * kb + (lane & 31)) * KROW + 8 * half];
#pragma unroll
            for (int st = 0; st < DS; ++st) {
                const fa_bf16x8_t kf = *reinterpret_cast<const fa_bf16x8_t*>(krow + 16 * st);
                s[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[st], s[kb], 0, 0, 0);
            }
        }

        // Masking is needed only on tiles that cross an end of some query's key
        // range in this wave: the end of the keys, a causal diagonal or a
        // segment bound (wave-uniform).
        const bool edge = t0 < wave_lo_max || t0 + FA_BN > wave_hi_min;
        float mt = -INFINITY;  // tile max of this query, log2 units
        if constexpr (MASK) {
            // an all-zero tile adds nothing: fmaf(0, log2 e, x) is x, so the mask is not read
            const bool zero = cls == FA_TILE_ZERO;
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const int key = t0 + 32 * kb + 8 * (e >> 2) + 4 * half + (e & 3);
                    const float mv = zero ? 0.0f : mrow[min(key, s_len - 1)];
                    float x = fmaf(mv, FA_LOG2E, s[kb][e] * a.scale_log2);
                    x = key >= rq.x && key < rq.y ? x : -INFINITY;
                    s[kb][e] = x;
                    mt = fmaxf(mt, x);
                }
            }
        } else {
            // raw scores stay unscaled: the scale (> 0) is applied to the max and
            // folded into the exponent below
            if (edge) {
#pragma unroll
                for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
                    for (int e = 0; e < 16; ++e) {
                        const int key = t0 + 32 * kb + 8 * (e >> 2) + 4 * half + (e & 3);
                        s[kb][e] = key >= rq.x && key < rq.y ? s[kb][e] : -INFINITY;
                    }
                }
            }
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                for (int e = 0; e < 16; ++e) mt = fmaxf(mt, s[kb][e]);
            mt *= a.scale_log2;
        }
        mt = xor_max<32>(mt);
        // The running max moves only when the tile's max exceeds it by more than
        // FA_RESCALE (log2 units): P then stays below 2^FA_RESCALE, and the O
        // rescale is skipped on the tiles where no lane of the wave needs it.
        const bool grow = mt > m_run + FA_RESCALE;
        const float m_new = grow ? mt : m_run;
        const bool none = m_new == -INFINITY;  // nothing visible yet: o and l stay zero
        const float alpha = grow && m_run != -INFINITY ? __builtin_amdgcn_exp2f(m_run - m_new) : (grow ? 0.0f : 1.0f);
        const float msub = none ? 0.0f : m_new;
        m_run = m_new;

        // P = 2^(S - m), packed to bf16 in k-slot order, and its sum
        const float sc = MASK ? 1.0f : a.scale_log2;
        uint32_t pk[2][8];
        float lsum = 0.0f;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
            for (int e = 0; e < 16; e += 2) {
                const float p0 = __builtin_amdgcn_exp2f(fmaf(s[kb][e], sc, -msub));
                const float p1 = __builtin_amdgcn_exp2f(fmaf(s[kb][e + 1], sc, -msub));
                lsum += p0 + p1;
                pk[kb][e / 2] = pack_bf16x2(p0, p1);
            }
        }
        l_part = fmaf(l_part, alpha, lsum);
        if (__builtin_amdgcn_ballot_w64(grow) != 0) {
#pragma unroll
            for (int i = 0; i < DB; ++i)
#pragma unroll
                for (int e = 0; e < 16; ++e) o[i][e] *= alpha;
        }

        // O^T += V^T . P^T: k-step (kb, stp) covers the keys of accumulator
        // entries 8 stp .. 8 stp + 7 of block kb:
        //   32 kb + 16 stp + 4 half + 0..3  and  32 kb + 16 stp + 8 + 4 half + 0..3
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
            for (int stp = 0; stp < 2; ++stp) {
                const fa_bf16x8_t pf =
                    as_bf16x8(pk[kb][4 * stp], pk[kb][4 * stp + 1], pk[kb][4 * stp + 2], pk[kb][4 * stp + 3]);
                // dims 32 db + lane % 32 of keys 32 kb + 16 stp + 4 half + 0..3 and + 8
                const uint16_t* vt = &vs[buf][v_lane + (32 * kb + 16 * stp) * VROW];
#pragma unroll
                for (int db = 0; db < DB; ++db) {
                    const uint2 va = lds_read_tr16_b64(vt + 32 * db);
                    const uint2 vb = lds_read_tr16_b64(vt + 8 * VROW + 32 * db);
                    o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(va.x, va.y, vb.x, vb.y), pf, o[db],
                                                                   0, 0, 0);
                }
            }
        }
        }  // cls != FA_TILE_MASKED: an all-masked tile contributes nothing and is skipped
        // the other buffer was last read in iteration t - 1, before the barrier that ended it
        if (t + 1 < t_end) store_tile(buf ^ 1);
        __syncthreads();
    }

    const float l = xor_sum<32>(l_part);
    const float inv = l > 0.0f ? 1.0f / l : 0.0f;
    if (q_valid) {
        uint16_t* orow = a.out + (size_t)b * a.o_sb + (size_t)qi * a.o_st + (size_t)h * a.o_sh;
#pragma unroll
        for (int db = 0; db < DB; ++db) {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int dim = 32 * db + 8 * g + 4 * half;
                const uint32_t lo = pack_bf16x2(o[db][4 * g] * inv, o[db][4 * g + 1] * inv);
                const uint32_t hi = pack_bf16x2(o[db][4 * g + 2] * inv, o[db][4 * g + 3] * inv);
                *reinterpret_cast<uint2*>(orow + dim) = make_uint2(lo, hi);
            }
        }
    }
}

// One block per (key tile, query block, mask batch): min and max of the mask over the block's FA_BM x FA_BN
// entries inside [t_len) x [s_len), then the class (FA_MASK_OPT_F16's rule).
__global__ __launch_bounds__(256) void fa_mask_tiles_kernel(const float* mask, size_t m_sb, size_t m_st,
                                                            uint32_t t_len, uint32_t s_len, uint32_t nqb,
                                                            uint32_t n_tiles, uint8_t* tiles) {
    const uint32_t tile = blockIdx.x, qb = blockIdx.y, b = blockIdx.z;
    float mn = FA_MASKED, mx = -FA_MASKED;
    for (uint32_t i = threadIdx.x; i < (uint32_t)(FA_BM * FA_BN); i += 256) {
        const uint32_t row = qb * FA_BM + i / FA_BN, col = tile * FA_BN + i % FA_BN;
        if (row < t_len && col < s_len) {
            const float v = mask[(size_t)b * m_sb + (size_t)row * m_st + col];
            mn = fminf(mn, v);
            mx = fmaxf(mx, v);
        }
    }
    mn = -wave_max(-mn);
    mx = wave_max(mx);
    __shared__ float rmn[4], rmx[4];
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
        rmn[wave] = mn;
        rmx[wave] = mx;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < 4; ++w) {
            mn = fminf(mn, rmn[w]);
            mx = fmaxf(mx, rmx[w]);
        }
        const uint8_t cls = mx <= -FA_MASKED ? FA_TILE_MASKED : (mn == 0.0f && mx == 0.0f ? FA_TILE_ZERO : FA_TILE_MIXED);
        tiles[((size_t)b * nqb + qb) * n_tiles + tile] = cls;
    }
}

template <int D>
static void fa_launch(bool causal, bool mask, bool seg, dim3 grid, const FaArgs& a, hipStream_t s) {
    const dim3 block(FA_THREADS);
    if (seg) {
        hipLaunchKernelGGL((fa_prefill_kernel<D, false, false, true>), grid, block, 0, s, a);
    } else if (causal) {
        if (mask) hipLaunchKernelGGL((fa_prefill_kernel<D, true, true, false>), grid, block, 0, s, a);
        else hipLaunchKernelGGL((fa_prefill_kernel<D, true, false, false>), grid, block, 0, s, a);
    } else {
        if (mask) hipLaunchKernelGGL((fa_prefill_kernel<D, false, true, false>), grid, block, 0, s, a);
        else hipLaunchKernelGGL((fa_prefill_kernel<D, false, false, false>), grid, block, 0, s, a);
    }
}

}  // namespace t2h

using namespace t2h;

static int fa_prefill(const void* q, const void* k, const void* v, void* out, const float* mask,
                      const uint8_t* tiles, const int32_t* cu, uint32_t n_seg, uint32_t batch, uint32_t nh,
                      uint32_t nk, uint32_t t_len, uint32_t s_len, uint32_t d, const int64_t* strides, int causal,
                      int32_t causal_offset, float scale, void* stream) {
    if (!q || !k || !v || !out || !strides) return T2H_ERR_NULL;
    if (d != 64 && d != 128) return T2H_ERR_UNSUPPORTED;
    if (nh == 0 || nk == 0 || nh % nk != 0) return T2H_ERR_SHAPE;
    if (batch == 0 || t_len == 0) return T2H_OK;
    if (s_len == 0) return T2H_ERR_SHAPE;
    // query blocks per (batch, head); with segments, a block per FA_BM tokens and one more per segment (the
    // blocks of each segment start at its first token), and one each for the tokens before and after the table
    const uint64_t nqb = cu ? (uint64_t)t_len / FA_BM + n_seg + 2 : ((uint64_t)t_len + FA_BM - 1) / FA_BM;
    if ((uint64_t)batch * nh * nqb > 0x7fffffffu || t_len > 0x7fffffffu - FA_BM || s_len > 0x7fffffffu)
        return T2H_ERR_SHAPE;
    const int n_strides = mask ? 14 : 12;
    for (int i = 0; i < n_strides; ++i)
        if (strides[i] < 0) return T2H_ERR_ARG;
    // 16-B q/k rows, 8-B v and out rows: pointers and (b, t, h) strides in elements
    const uintptr_t align_bits = reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k);
    if ((align_bits & 15) != 0 || (reinterpret_cast<uintptr_t>(v) & 7) != 0 ||
        (reinterpret_cast<uintptr_t>(out) & 7) != 0)
        return T2H_ERR_ALIGN;
    for (int i = 0; i < 6; ++i)
        if (strides[i] % 8 != 0) return T2H_ERR_ALIGN;
    for (int i = 6; i < 12; ++i)
        if (strides[i] % 4 != 0) return T2H_ERR_ALIGN;
    // a tile's key rows are addressed by 32-bit element offsets from its first row
    if ((uint64_t)FA_BN * (uint64_t)(strides[4] > strides[7] ? strides[4] : strides[7]) + d > 0xffffffffu)
        return T2H_ERR_SHAPE;
    FaArgs a = {};
    a.q = reinterpret_cast<const uint16_t*>(q);
    a.k = reinterpret_cast<const uint16_t*>(k);
    a.v = reinterpret_cast<const uint16_t*>(v);
    a.out = reinterpret_cast<uint16_t*>(out);
    a.mask = mask;
    a.cu = cu;
    a.n_seg = n_seg;
    a.q_sb = (size_t)strides[0];
    a.q_st = (size_t)strides[1];
    a.q_sh = (size_t)strides[2];
    a.k_sb = (size_t)strides[3];
    a.k_st = (size_t)strides[4];
    a.k_sh = (size_t)strides[5];
    a.v_sb = (size_t)strides[6];
    a.v_st = (size_t)strides[7];
    a.v_sh = (size_t)strides[8];
    a.o_sb = (size_t)strides[9];
    a.o_st = (size_t)strides[10];
    a.o_sh = (size_t)strides[11];
    if (mask) {
        a.m_sb = (size_t)strides[12];
        a.m_st = (size_t)strides[13];
        a.tiles = tiles;
        a.n_tiles = (s_len + FA_BN - 1) / FA_BN;
        a.tiles_sb = a.m_sb == 0 ? 0 : (size_t)((t_len + FA_BM - 1) / FA_BM) * a.n_tiles;
    }
    a.nh = nh;
    a.group = nh / nk;
    a.batch = batch;
    a.t_len = t_len;
    a.s_len = s_len;
    a.causal_offset = causal_offset;
    const float sc = scale > 0.0f ? scale : 1.0f / sqrtf((float)d);
    a.scale_log2 = sc * FA_LOG2E;
    const dim3 grid((uint32_t)(nqb * batch * nh));
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    if (d == 128) fa_launch<128>(causal != 0, mask != nullptr, cu != nullptr, grid, a, s);
    else fa_launch<64>(causal != 0, mask != nullptr, cu != nullptr, grid, a, s);
    T2H_LAUNCH_CHECK();
    return T2H_OK;
}

extern "C" int t2h_flash_attn_prefill(const void* q, const void* k, const void* v, void* out, const float* mask,
                                      uint32_t batch, uint32_t nh, uint32_t nk, uint32_t t_len, uint32_t s_len,
                                      uint32_t d, const int64_t* strides, int causal, int32_t causal_offset,
                                      float scale, void* stream) {
    return fa_prefill(q, k, v, out, mask, nullptr, nullptr, 0, batch, nh, nk, t_len, s_len, d, strides, causal,
                      causal_offset, scale, stream);
}

extern "C" int t2h_flash_attn_prefill_tiles(const void* q, const void* k, const void* v, void* out,
                                            const float* mask, const uint8_t* mask_tiles, uint32_t batch,
                                            uint32_t nh, uint32_t nk, uint32_t t_len, uint32_t s_len, uint32_t d,
                                            const int64_t* strides, int causal, int32_t causal_offset, float scale,
                                            void* stream) {
    if (!mask || !mask_tiles) return T2H_ERR_NULL;
    return fa_prefill(q, k, v, out, mask, mask_tiles, nullptr, 0, batch, nh, nk, t_len, s_len, d, strides, causal,
                      causal_offset, scale, stream);
}

extern "C" int t2h_fa_mask_tiles(const float* mask, uint32_t mask_batch, uint32_t t_len, uint32_t s_len,
                                 int64_t m_sb, int64_t m_st, uint8_t* tiles, void* stream) {
    if (!mask || !tiles) return T2H_ERR_NULL;
    if (m_sb < 0 || m_st < 0) return T2H_ERR_ARG;
    if (mask_batch == 0 || t_len == 0 || s_len == 0) return T2H_OK;
    const uint32_t nqb = (t_len + FA_BM - 1) / FA_BM, n_tiles = (s_len + FA_BN - 1) / FA_BN;
    if (mask_batch > 65535u || nqb > 65535u) return T2H_ERR_SHAPE;
    hipLaunchKernelGGL(fa_mask_tiles_kernel, dim3(n_tiles, nqb, mask_batch), dim3(256), 0,
                       reinterpret_cast<hipStream_t>(stream), mask, (size_t)m_sb, (size_t)m_st, t_len, s_len, nqb,
                       n_tiles, tiles);
    T2H_LAUNCH_CHECK();
    return T2H_OK;
}

extern "C" int t2h_flash_attn_segments(const void* q, const void* k, const void* v, void* out,
                                       const int32_t* cu_seqlens, uint32_t n_seg, uint32_t batch, uint32_t nh,
                                       uint32_t nk, uint32_t t_len, uint32_t d, const int64_t* strides, float scale,
                                       void* stream) {
    if (!cu_seqlens) return T2H_ERR_NULL;
    if (n_seg == 0 || n_seg > 0x7fffffffu) return T2H_ERR_SHAPE;
    return fa_prefill(q, k, v, out, nullptr, nullptr, cu_seqlens, n_seg, batch, nh, nk, t_len, t_len, d, strides, 0,
                      0, scale, stream);
}
