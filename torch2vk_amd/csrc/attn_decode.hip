// Split-K decode attention (flash-decoding) over a token-major GQA KV cache.
//
// Replaces, for one decode token:
//   RMS_NORM_ROPE_TRANSPOSE_F16 x2 (q-norm, k-norm + RoPE)
//       src/models/optimized_qwen3/shaders/rms_norm_rope_transpose_f16.py:22-145
//   ROPE_TABLE_F32 (cos/sin at cache_position)        src/torch2vk/runtime/rope_table.py:32-122
//   SDPA_DECODE_CACHE_WRITE_F32 (cache write + attention)
//       src/models/optimized_qwen3/shaders/sdpa_decode_cache_write_f32.py:22-170
//
// The reference walks the whole cache serially in one workgroup per q head.
// Here the grid is fixed at (slots, nk) with slots * nk = 256 blocks, one per
// CU, whatever the length: block (slot, kv head) has W waves (8; 4 at GROUP 8)
// and wave w covers span = ceil(L / (slots * W)) consecutive positions for all
// GROUP q heads of the kv head, so every K/V byte is read once per token and
// every CU streams an equal share:
//   * K rows are loaded coalesced (4 lanes per row, 64 B each, 16 rows per
//     load set) and a lane dots its quarter row with the GROUP q vectors
//     (broadcast from LDS); a quad DPP reduction completes the dot;
//   * V is loaded coalesced straight into registers in the P.V layout (lane
//     owns two dims, one register per position);
//   * a wave walks its span in tiles of 32 positions with an online softmax
//     (one tile up to L = 8192 at 256 blocks), loading only rows < L;
//   * the waves' partial softmax states are merged in LDS and the block's
//     (max, sum, unnormalised output) is published to the workspace;
//   * a second small kernel merges the slots' partials of each q head with the
//     log-sum-exp rule.  Merging in the last block to finish would need
//     device-scope release/acquire: on this multi-XCD part that is an L2
//     write-back plus invalidate per block, measured far slower than a launch.
//
// Cache layout (as the reference's optimized decode cache): bf16
// [S_cap, NK, D], token-major.  q/k/v inputs are the fp32 QKV projections.
// The current position is read from device memory, so a captured graph can
// replay the step with an advancing position.
#include "common.h"
#include "rope.h"

namespace t2h {

constexpr int AD_D = 128;
constexpr int AD_WAVES = 8;                   // waves per block (4 for GROUP 8, see ad_waves)
constexpr int AD_TILE = 32;                   // positions per wave per tile (two 16-row K load sets; 16 for GROUP 8)
constexpr int AD_GRID = 256;                  // split blocks per call (slots * nk), one per CU
constexpr int AD_QROW = 36;                   // LDS q row: 32 dims + 4 pad (conflict-free quarter reads)
constexpr int AD_MERGE_WAVES = 4;
constexpr int AD_MERGE_BATCH = 16;            // partial loads in flight per merge wave

struct AttnDecodeArgs {
    const float* q;         // [NH, D] fp32
    const float* k_new;     // [NK, D] fp32
    const float* v_new;     // [NK, D] fp32
    const float* q_norm_w;  // [D] or null (inputs already normalised)
    const float* k_norm_w;  // [D] or null
    uint16_t* k_cache;      // bf16 [S_cap, NK, D]
    uint16_t* v_cache;
    uint16_t* out;          // bf16 [NH, D]
    const int32_t* pos_ptr; // current position (device)
    float* part_ml;         // [NK, slots, GROUP, 2]
    float* part_o;          // [NK, slots, GROUP, D]
    uint32_t nk;
    uint32_t s_cap;
    uint32_t slots;         // split blocks per kv head
    float theta;            // <= 0: no RoPE
    float eps;
    float scale;            // softmax scale, 1/sqrt(D)
};

// K and V rows of one tile: positions t + 16 r + p_k of the K quarter `part`,
// and V rows t .. t + TILE - 1 (lane owns dims 2 lane, 2 lane + 1).
template <int TILE>
struct AdTile {
    uint4 kr[TILE / 16][4];
    uint32_t vr[TILE];
};

// Load the rows [t, t + n) of a tile (n >= 1, wave-uniform).  K lanes past the
// end re-read row t + n - 1 (always valid) instead of branching, so all loads
// of the tile are in flight at once; V rows past the end are not loaded.
template <int TILE>
__device__ __forceinline__ void ad_issue_tile(AdTile<TILE>& tl, const uint16_t* kbase, const uint16_t* vbase,
                                              size_t row_stride, int t, int n) {
    const int lane = threadIdx.x & 63;
    const int p_k = lane >> 2, part = lane & 3;
#pragma unroll
    for (int r = 0; r < TILE / 16; ++r) {
        if (r == 0 || n > 16 * r) {
            const int p = t + min(16 * r + p_k, n - 1);
            const uint16_t* krow = kbase + (size_t)p * row_stride + part * 32;
#pragma unroll
            for (int i = 0; i < 4; ++i) tl.kr[r][i] = load_u4(krow + 8 * i);
        }
    }
#pragma unroll
    for (int i = 0; i < TILE; ++i)
        if (i < n) tl.vr[i] = reinterpret_cast<const uint32_t*>(vbase + (size_t)(t + i) * row_stride)[lane];
}

// Split-K pass: see the file comment.  Block (slot, kv head); the new K/V row
// at `pos` is produced by the wave whose span holds it, written to the cache
// and substituted for the (stale) row it loaded.
// Waves per split block.  At GROUP 8 a wave carries 8 heads' running state beside its tile, which does not fit
// the 256 registers of two waves per SIMD: that instantiation runs 4 waves, one per SIMD with the whole
// register file, each preparing q heads wave and wave + 4.
template <int GROUP>
constexpr int ad_waves() { return GROUP >= 8 ? 4 : AD_WAVES; }

template <int GROUP>
__global__ __launch_bounds__(ad_waves<GROUP>() * 64) void attn_decode_kernel(const AttnDecodeArgs a) {
    constexpr int W = ad_waves<GROUP>();
    constexpr int QH = (GROUP + W - 1) / W;           // q heads prepared per wave: wave, wave + W, ...
    constexpr int TILE = GROUP >= 8 ? 16 : AD_TILE;  // registers: TILE V rows + GROUP accumulators
    constexpr int NR = TILE / 16;                     // 16-row K load sets per tile
    __shared__ __align__(16) float qs[GROUP][4][AD_QROW];
    __shared__ __align__(16) float ps[W][TILE][GROUP];
    __shared__ float wml[W][GROUP][2];
    __shared__ __align__(16) float2 wo[W][GROUP][64];
    __shared__ __align__(16) uint16_t knew[AD_D];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform, scalar
    const int slot = blockIdx.x;
    const int kvh = blockIdx.y;
    const int pos = *a.pos_ptr;
    const int S = (int)a.s_cap;
    const int L = pos + 1 < S ? pos + 1 : S;
    const int waves_per_head = (int)a.slots * W;
    const int span = (L + waves_per_head - 1) / waves_per_head;
    const int pw = (slot * W + wave) * span;  // first position of this wave
    int rows = L - pw;
    rows = rows < 0 ? 0 : (rows > span ? span : rows);
    const size_t row_stride = (size_t)a.nk * AD_D;  // elements between positions
    const uint16_t* kbase = a.k_cache + (size_t)kvh * AD_D;
    const uint16_t* vbase = a.v_cache + (size_t)kvh * AD_D;
    const bool has_new = pos < S && pos >= pw && pos < pw + rows;  // wave-uniform
    const bool rope = a.theta > 0.0f;
    const bool needs_rope = wave < GROUP || has_new;  // wave-uniform

    // 0. the small operands first: vmcnt retires in order, so anything loaded
    //    after the cache stream would wait for all of it
    const bool has_w = a.q_norm_w != nullptr;
    float qx0[QH], qx1[QH];
#pragma unroll
    for (int i = 0; i < QH; ++i) {
        qx0[i] = qx1[i] = 0.0f;
        if (wave + i * W < GROUP) {
            const int h = kvh * GROUP + wave + i * W;
            qx0[i] = a.q[h * AD_D + lane];
            qx1[i] = a.q[h * AD_D + lane + 64];
        }
    }
    float qw0 = 1.0f, qw1 = 1.0f, kw0 = 1.0f, kw1 = 1.0f;
    if (has_w && needs_rope) {
        qw0 = a.q_norm_w[lane];
        qw1 = a.q_norm_w[lane + 64];
        kw0 = a.k_norm_w[lane];
        kw1 = a.k_norm_w[lane + 64];
    }
    float kx0 = 0.0f, kx1 = 0.0f, vx0 = 0.0f, vx1 = 0.0f;
    if (has_new) {
        kx0 = a.k_new[kvh * AD_D + lane];
        kx1 = a.k_new[kvh * AD_D + lane + 64];
        vx0 = a.v_new[kvh * AD_D + 2 * lane];
        vx1 = a.v_new[kvh * AD_D + 2 * lane + 1];
    }

    // 1. the first tile's K/V rows
    AdTile<TILE> tl;
    if (rows > 0) ad_issue_tile(tl, kbase, vbase, row_stride, pw, min(rows, TILE));

    // 2. RoPE at `pos` (lane = frequency index, inv_freq = theta^(-2 lane / D));
    //    q head `wave` normalised, rotated, pre-scaled by 1/sqrt(D) into LDS
    float cs = 1.0f, sn = 0.0f;
    if (rope && needs_rope) {
        rope_cos_sin(lane, pos, a.theta, cs, sn);
    }
#pragma unroll
    for (int i = 0; i < QH; ++i) {
        const int g = wave + i * W;
        if (g < GROUP) {
            float r0, r1;
            norm_rope_pair(qx0[i], qx1[i], has_w, qw0, qw1, a.eps, cs, sn, rope, r0, r1);
            qs[g][lane >> 5][lane & 31] = r0 * a.scale;
            qs[g][2 + (lane >> 5)][lane & 31] = r1 * a.scale;
        }
    }

    // 3. the wave holding `pos` produces the new K/V row and writes it back
    uint32_t vnew = 0;
    if (has_new) {
        float k0, k1;
        norm_rope_pair(kx0, kx1, has_w, kw0, kw1, a.eps, cs, sn, rope, k0, k1);
        const uint16_t kb0 = (uint16_t)f32_to_bf16_bits(k0);
        const uint16_t kb1 = (uint16_t)f32_to_bf16_bits(k1);
        knew[lane] = kb0;
        knew[lane + 64] = kb1;
        vnew = pack_bf16x2(vx0, vx1);
        const size_t off = (size_t)pos * row_stride + (size_t)kvh * AD_D;
        a.k_cache[off + lane] = kb0;
        a.k_cache[off + lane + 64] = kb1;
        reinterpret_cast<uint32_t*>(a.v_cache + off)[lane] = vnew;
    }
    __syncthreads();

    // 4. tiles: scores, online softmax, P.V (a wave with no rows keeps m = -inf, l = 0, o = 0)
    const int p_k = lane >> 2;
    const int part = lane & 3;
    float mg[GROUP], lg[GROUP], o0[GROUP], o1[GROUP];
#pragma unroll
    for (int g = 0; g < GROUP; ++g) {
        mg[g] = -INFINITY;
        lg[g] = 0.0f;
        o0[g] = o1[g] = 0.0f;
    }
    // one tile: rows [t0, t0 + n) of the wave's span, loaded into tl
    auto tile = [&](AdTile<TILE>& tl, int t0, int n) {
        const int tnew = pos - (pw + t0);  // row of the new position within the tile (if any)
        float s[NR][GROUP];
#pragma unroll
        for (int r = 0; r < NR; ++r) {
            if (has_new && 16 * r + p_k == tnew) {
#pragma unroll
                for (int i = 0; i < 4; ++i) tl.kr[r][i] = *reinterpret_cast<const uint4*>(&knew[part * 32 + 8 * i]);
            }
#pragma unroll
            for (int g = 0; g < GROUP; ++g) s[r][g] = 0.0f;
        }
        // each q fragment read from LDS once and used for both K rows
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float kf[NR][8];
#pragma unroll
            for (int r = 0; r < NR; ++r) {
                const uint4 kk = tl.kr[r][i];
                kf[r][0] = bf16_bits_to_f32(kk.x & 0xffffu); kf[r][1] = bf16_bits_to_f32(kk.x >> 16);
                kf[r][2] = bf16_bits_to_f32(kk.y & 0xffffu); kf[r][3] = bf16_bits_to_f32(kk.y >> 16);
                kf[r][4] = bf16_bits_to_f32(kk.z & 0xffffu); kf[r][5] = bf16_bits_to_f32(kk.z >> 16);
                kf[r][6] = bf16_bits_to_f32(kk.w & 0xffffu); kf[r][7] = bf16_bits_to_f32(kk.w >> 16);
            }
#pragma unroll
            for (int g = 0; g < GROUP; ++g) {
                const float4 qa = *reinterpret_cast<const float4*>(&qs[g][part][8 * i]);
                const float4 qb = *reinterpret_cast<const float4*>(&qs[g][part][8 * i + 4]);
#pragma unroll
                for (int r = 0; r < NR; ++r) {
                    float u = s[r][g];
                    u = fmaf(qa.x, kf[r][0], u); u = fmaf(qa.y, kf[r][1], u);
                    u = fmaf(qa.z, kf[r][2], u); u = fmaf(qa.w, kf[r][3], u);
                    u = fmaf(qb.x, kf[r][4], u); u = fmaf(qb.y, kf[r][5], u);
                    u = fmaf(qb.z, kf[r][6], u); u = fmaf(qb.w, kf[r][7], u);
                    s[r][g] = u;
                }
            }
        }
#pragma unroll
        for (int g = 0; g < GROUP; ++g) {
            float sc[NR];
            float tmax = -INFINITY;
#pragma unroll
            for (int r = 0; r < NR; ++r) {
                float u = s[r][g];
                u += dpp_f32<0xB1>(u);  // quad_perm [1,0,3,2]
                u += dpp_f32<0x4E>(u);  // quad_perm [2,3,0,1]
                sc[r] = 16 * r + p_k < n ? u : -INFINITY;
                tmax = fmaxf(tmax, sc[r]);
            }
            const float m = fmaxf(mg[g], wave_max(tmax));  // finite: the tile has >= 1 row
            const float rescale = mg[g] == -INFINITY ? 0.0f : expf(mg[g] - m);
            float esum = 0.0f;
#pragma unroll
            for (int r = 0; r < NR; ++r) {
                const float e = 16 * r + p_k < n ? expf(sc[r] - m) : 0.0f;
                esum += e;
                if (part == 0) ps[wave][16 * r + p_k][g] = e;
            }
            mg[g] = m;
            lg[g] = fmaf(lg[g], rescale, wave_sum(part == 0 ? esum : 0.0f));
            o0[g] *= rescale;
            o1[g] *= rescale;
        }
        // ps is produced and consumed by the same wave: LDS order within a wave suffices
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        // P.V: lane <-> dims (2 lane, 2 lane + 1), V from registers (fully
        // unrolled so they are indexed statically; rows >= n are skipped).  The
        // scheduling fence every 8 rows keeps the P reads from all being hoisted
        // into registers at once.
#pragma unroll
        for (int p = 0; p < TILE; ++p) {
            if (p % 8 == 0) __builtin_amdgcn_sched_barrier(0);
            if (p < n) {
                const uint32_t vv = (has_new && p == tnew) ? vnew : tl.vr[p];
                const float va = bf16_bits_to_f32(vv & 0xffffu);
                const float vb = bf16_bits_to_f32(vv >> 16);
#pragma unroll
                for (int g = 0; g < GROUP; ++g) {
                    const float pr = ps[wave][p][g];
                    o0[g] = fmaf(pr, va, o0[g]);
                    o1[g] = fmaf(pr, vb, o1[g]);
                }
            }
        }
        __builtin_amdgcn_wave_barrier();  // the next tile's ps writes come after these reads
    };
    // the first tile was loaded before the q preparation; tiles past it (spans
    // over 32 rows: L > 8192 at 256 blocks) load and then compute
    if (rows > 0) tile(tl, 0, min(rows, TILE));
    for (int t0 = TILE; t0 < rows; t0 += TILE) {
        const int n = min(rows - t0, TILE);
        AdTile<TILE> tn;
        ad_issue_tile(tn, kbase, vbase, row_stride, pw + t0, n);
        tile(tn, t0, n);
    }

    // 5. merge the waves in LDS and publish the block's partial
#pragma unroll
    for (int g = 0; g < GROUP; ++g) {
        wo[wave][g][lane] = make_float2(o0[g], o1[g]);
        if (lane == 0) {
            wml[wave][g][0] = mg[g];
            wml[wave][g][1] = lg[g];
        }
    }
    __syncthreads();
    const size_t cbase = ((size_t)kvh * a.slots + slot) * GROUP;  // first partial of this block
    for (int idx = tid; idx < GROUP * 64; idx += W * 64) {
        const int g = idx >> 6;
        const int dl = idx & 63;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < W; ++w) M = fmaxf(M, wml[w][g][0]);
        float l = 0.0f, r0 = 0.0f, r1 = 0.0f;
#pragma unroll
        for (int w = 0; w < W; ++w) {
            const float m = wml[w][g][0];
            const float f = m == -INFINITY ? 0.0f : expf(m - M);
            l = fmaf(f, wml[w][g][1], l);
            const float2 ov = wo[w][g][dl];
            r0 = fmaf(f, ov.x, r0);
            r1 = fmaf(f, ov.y, r1);
        }
        *reinterpret_cast<float2*>(&a.part_o[(cbase + g) * AD_D + 2 * dl]) = make_float2(r0, r1);
        if (dl == 0) *reinterpret_cast<float2*>(&a.part_ml[(cbase + g) * 2]) = make_float2(M, l);
    }
}

// Log-sum-exp merge of the per-slot partials: one block per q head, each of
// its AD_MERGE_WAVES waves folds a slab of up to AD_MERGE_BATCH chunks at a
// time (loads issued together; indices past the end re-read the last chunk and
// get weight 0), then the waves' states are combined in LDS.  Lane t owns dims
// 2t and 2t+1.
template <int GROUP>
__global__ __launch_bounds__(AD_MERGE_WAVES * 64) void attn_decode_merge_kernel(const AttnDecodeArgs a) {
    __shared__ float fs[AD_MERGE_WAVES][AD_MERGE_BATCH];
    __shared__ float wst[AD_MERGE_WAVES][2];
    __shared__ float2 wacc[AD_MERGE_WAVES][64];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int h = blockIdx.x;
    const int kvh = h / GROUP;
    const int g = h % GROUP;
    const int n_chunks = (int)a.slots;  // every slot publishes a partial (m = -inf, l = 0 when it saw no row)
    const size_t hbase = (size_t)kvh * a.slots * GROUP + g;
    float M = -INFINITY, lsum = 0.0f, acc0 = 0.0f, acc1 = 0.0f;
    for (int cb = wave * AD_MERGE_BATCH; cb < n_chunks; cb += AD_MERGE_WAVES * AD_MERGE_BATCH) {
        float2 ov[AD_MERGE_BATCH];
        float mv = -INFINITY, lv = 0.0f;
        if (lane < AD_MERGE_BATCH) {
            const int cc = min(cb + lane, n_chunks - 1);
            const float2 ml = load_nt_f2(&a.part_ml[(hbase + (size_t)cc * GROUP) * 2]);
            if (cb + lane < n_chunks) {
                mv = ml.x;
                lv = ml.y;
            }
        }
#pragma unroll
        for (int i = 0; i < AD_MERGE_BATCH; ++i) {
            const int cc = min(cb + i, n_chunks - 1);
            ov[i] = load_nt_f2(&a.part_o[(hbase + (size_t)cc * GROUP) * AD_D + 2 * lane]);
        }
        const float mb = fmaxf(M, wave_max(mv));
        const float rescale = M == -INFINITY ? 0.0f : expf(M - mb);
        const float f = mv == -INFINITY ? 0.0f : expf(mv - mb);
        lsum = lsum * rescale + wave_sum(f * lv);
        acc0 *= rescale;
        acc1 *= rescale;
        M = mb;
        if (lane < AD_MERGE_BATCH) fs[wave][lane] = f;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (int i = 0; i < AD_MERGE_BATCH; ++i) {
            acc0 = fmaf(fs[wave][i], ov[i].x, acc0);
            acc1 = fmaf(fs[wave][i], ov[i].y, acc1);
        }
        __builtin_amdgcn_wave_barrier();
    }
    wacc[wave][lane] = make_float2(acc0, acc1);
    if (lane == 0) {
        wst[wave][0] = M;
        wst[wave][1] = lsum;
    }
    __syncthreads();
    if (wave == 0) {
        float Mt = -INFINITY;
#pragma unroll
        for (int w = 0; w < AD_MERGE_WAVES; ++w) Mt = fmaxf(Mt, wst[w][0]);
        float lt = 0.0f, r0 = 0.0f, r1 = 0.0f;
#pragma unroll
        for (int w = 0; w < AD_MERGE_WAVES; ++w) {
            const float f = wst[w][0] == -INFINITY ? 0.0f : expf(wst[w][0] - Mt);
            lt = fmaf(f, wst[w][1], lt);
            r0 = fmaf(f, wacc[w][lane].x, r0);
            r1 = fmaf(f, wacc[w][lane].y, r1);
        }
        const float inv = 1.0f / lt;
        reinterpret_cast<uint32_t*>(a.out)[(h * AD_D) / 2 + lane] = pack_bf16x2(r0 * inv, r1 * inv);
    }
}

}  // namespace t2h

using namespace t2h;

// split blocks per kv head: AD_GRID blocks in all (one per CU), at least one per kv head
static uint32_t ad_slots(uint32_t nk) { return nk >= (uint32_t)AD_GRID ? 1u : (uint32_t)AD_GRID / nk; }

static size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

extern "C" size_t t2h_attn_decode_workspace_bytes(uint32_t nh, uint32_t nk, uint32_t d, uint32_t s_cap) {
    if (nk == 0 || nh % nk != 0 || d != AD_D || s_cap == 0 || s_cap > (uint32_t)INT32_MAX) return 0;
    const size_t parts = (size_t)nk * ad_slots(nk) * (nh / nk);
    return align256(parts * 2 * sizeof(float)) + align256(parts * d * sizeof(float));
}

extern "C" int t2h_attn_decode(const float* q, const float* k_new, const float* v_new, const float* q_norm_w,
                               const float* k_norm_w, float eps, float theta, void* k_cache, void* v_cache,
                               void* out, uint32_t nh, uint32_t nk, uint32_t d, uint32_t s_cap,
                               const int32_t* cache_position, void* workspace, size_t workspace_bytes,
                               void* stream) {
    if (!q || !k_new || !v_new || !k_cache || !v_cache || !out || !cache_position || !workspace) return T2H_ERR_NULL;
    if (d != AD_D) return T2H_ERR_UNSUPPORTED;
    if (nk == 0 || nh == 0 || nh % nk != 0 || s_cap == 0) return T2H_ERR_SHAPE;
    if (s_cap > (uint32_t)INT32_MAX) return T2H_ERR_UNSUPPORTED;
    if ((q_norm_w == nullptr) != (k_norm_w == nullptr)) return T2H_ERR_ARG;
    const uint32_t group = nh / nk;
    if (workspace_bytes < t2h_attn_decode_workspace_bytes(nh, nk, d, s_cap)) return T2H_ERR_WORKSPACE;
    const uint32_t slots = ad_slots(nk);
    AttnDecodeArgs a;
    a.q = q;
    a.k_new = k_new;
    a.v_new = v_new;
    a.q_norm_w = q_norm_w;
    a.k_norm_w = k_norm_w;
    a.k_cache = reinterpret_cast<uint16_t*>(k_cache);
    a.v_cache = reinterpret_cast<uint16_t*>(v_cache);
    a.out = reinterpret_cast<uint16_t*>(out);
    a.pos_ptr = cache_position;
    uint8_t* ws = reinterpret_cast<uint8_t*>(workspace);
    a.part_ml = reinterpret_cast<float*>(ws);
    ws += align256((size_t)nk * slots * group * 2 * sizeof(float));
    a.part_o = reinterpret_cast<float*>(ws);
    a.nk = nk;
    a.s_cap = s_cap;
    a.slots = slots;
    a.theta = theta;
    a.eps = eps;
    a.scale = 1.0f / sqrtf((float)d);
    const dim3 grid(slots, nk);
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const dim3 mgrid(nh), mblock(AD_MERGE_WAVES * 64);
    switch (group) {
#define T2H_AD_CASE(G)                                                                   \
    case G:                                                                              \
        hipLaunchKernelGGL(attn_decode_kernel<G>, grid, dim3(ad_waves<G>() * 64), 0, s, a); \
        T2H_LAUNCH_CHECK();                                                              \
        hipLaunchKernelGGL(attn_decode_merge_kernel<G>, mgrid, mblock, 0, s, a);         \
        break;
        T2H_AD_CASE(1)
        T2H_AD_CASE(2)
        T2H_AD_CASE(4)
        T2H_AD_CASE(8)
#undef T2H_AD_CASE
        default:
            return T2H_ERR_UNSUPPORTED;
    }
    T2H_LAUNCH_CHECK();
    return T2H_OK;
}
