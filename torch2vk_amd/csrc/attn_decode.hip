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
// Here a block owns (kv head, 64-position chunk): it stages the chunk's K and
// V rows in LDS once for all GROUP q heads of the kv head, computes a partial
// softmax (max, sum, unnormalised output), and the last block of each kv
// head to finish (atomic ticket) merges the partials with the log-sum-exp
// rule and resets its ticket, so a single launch is graph-replayable.
//
// Cache layout (as the reference's optimized decode cache): bf16
// [S_cap, NK, D], token-major.  q/k/v inputs are the fp32 QKV projections.
// The current position is read from device memory, so a captured graph can
// replay the step with an advancing position.
#include "common.h"

namespace t2h {

constexpr int AD_D = 128;
constexpr int AD_CH = 64;    // positions per block
constexpr int AD_KROW = 68;  // LDS K row stride in dwords (256 B + 16 B pad: conflict-free column reads)

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
    uint32_t* tickets;      // [NK]
    float* part_ml;         // [NK, max_chunks, GROUP, 2]
    float* part_o;          // [NK, max_chunks, GROUP, D]
    uint32_t nk;
    uint32_t s_cap;
    uint32_t max_chunks;
    float theta;            // <= 0: no RoPE
    float eps;
    float scale;            // softmax scale, 1/sqrt(D)
};

__device__ __forceinline__ void norm_rope_pair(float x0, float x1, const float* w, int lane, float eps, float cs,
                                               float sn, bool rope, float& r0, float& r1) {
    float n0 = x0, n1 = x1;
    if (w) {
        const float ss = wave_sum(x0 * x0 + x1 * x1);
        const float inv = 1.0f / sqrtf(ss / (float)AD_D + eps);
        n0 = x0 * inv * w[lane];
        n1 = x1 * inv * w[lane + 64];
    }
    if (rope) {
        // rotate_half pairs d with d + D/2: out[d] = n[d]cos - n[d+D/2]sin, out[d+D/2] = n[d+D/2]cos + n[d]sin
        r0 = n0 * cs - n1 * sn;
        r1 = n1 * cs + n0 * sn;
    } else {
        r0 = n0;
        r1 = n1;
    }
}

template <int GROUP>
__global__ __launch_bounds__(64) void attn_decode_kernel(const AttnDecodeArgs a) {
    __shared__ __align__(16) uint32_t ks[AD_CH * AD_KROW];
    __shared__ __align__(16) uint32_t vs[AD_CH * (AD_D / 2)];
    __shared__ __align__(16) float qs[GROUP][AD_D];
    __shared__ __align__(16) float ps[AD_CH][GROUP];

    const int lane = threadIdx.x;
    const int c = blockIdx.x;
    const int kvh = blockIdx.y;
    const int pos = *a.pos_ptr;
    const int S = (int)a.s_cap;
    const int L = pos + 1 < S ? pos + 1 : S;
    const int n_chunks = (L + AD_CH - 1) / AD_CH;
    if (c >= n_chunks) return;
    const int p0 = c * AD_CH;
    const int rows = (L - p0) < AD_CH ? (L - p0) : AD_CH;
    const size_t row_stride = (size_t)a.nk * AD_D;  // elements between positions

    // 1. issue the chunk's K/V loads: 4 rows per instruction, 16 B per lane
    uint4 kr[16], vr[16];
    const int rsub = lane >> 4;
    const int col = (lane & 15) * 8;  // bf16 element offset within the row
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int r = i * 4 + rsub;
        if (r < rows) {
            const size_t off = (size_t)(p0 + r) * row_stride + (size_t)kvh * AD_D + col;
            kr[i] = load_nt_u4(a.k_cache + off);
            vr[i] = load_nt_u4(a.v_cache + off);
        } else {
            kr[i] = make_uint4(0, 0, 0, 0);
            vr[i] = make_uint4(0, 0, 0, 0);
        }
    }

    // 2. q: per-head RMSNorm + RoPE at `pos`, pre-scaled by 1/sqrt(D)
    const bool rope = a.theta > 0.0f;
    float cs = 1.0f, sn = 0.0f;
    if (rope) {
        const float exponent = (2.0f * (float)lane) / (float)AD_D;
        const float inv_freq = powf(a.theta, -exponent);
        const float angle = (float)pos * inv_freq;
        sincosf(angle, &sn, &cs);
    }
#pragma unroll
    for (int g = 0; g < GROUP; ++g) {
        const int h = kvh * GROUP + g;
        float r0, r1;
        norm_rope_pair(a.q[h * AD_D + lane], a.q[h * AD_D + lane + 64], a.q_norm_w, lane, a.eps, cs, sn, rope, r0, r1);
        qs[g][lane] = r0 * a.scale;
        qs[g][lane + 64] = r1 * a.scale;
    }

    // 3. stage K/V in LDS
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int r = i * 4 + rsub;
        *reinterpret_cast<uint4*>(&ks[r * AD_KROW + (lane & 15) * 4]) = kr[i];
        *reinterpret_cast<uint4*>(&vs[r * (AD_D / 2) + (lane & 15) * 4]) = vr[i];
    }

    // 4. the chunk holding `pos` produces the new K/V row and writes it back
    if (pos < S && pos >= p0 && pos < p0 + AD_CH) {
        const int r = pos - p0;
        float k0, k1;
        norm_rope_pair(a.k_new[kvh * AD_D + lane], a.k_new[kvh * AD_D + lane + 64], a.k_norm_w, lane, a.eps, cs, sn,
                       rope, k0, k1);
        const uint16_t kb0 = (uint16_t)f32_to_bf16_bits(k0);
        const uint16_t kb1 = (uint16_t)f32_to_bf16_bits(k1);
        const uint16_t vb0 = (uint16_t)f32_to_bf16_bits(a.v_new[kvh * AD_D + lane]);
        const uint16_t vb1 = (uint16_t)f32_to_bf16_bits(a.v_new[kvh * AD_D + lane + 64]);
        uint16_t* krow = reinterpret_cast<uint16_t*>(&ks[r * AD_KROW]);
        uint16_t* vrow = reinterpret_cast<uint16_t*>(&vs[r * (AD_D / 2)]);
        krow[lane] = kb0;
        krow[lane + 64] = kb1;
        vrow[lane] = vb0;
        vrow[lane + 64] = vb1;
        const size_t off = (size_t)pos * row_stride + (size_t)kvh * AD_D;
        a.k_cache[off + lane] = kb0;
        a.k_cache[off + lane + 64] = kb1;
        a.v_cache[off + lane] = vb0;
        a.v_cache[off + lane + 64] = vb1;
    }
    __syncthreads();

    // 5. scores: lane <-> position
    float s[GROUP];
#pragma unroll
    for (int g = 0; g < GROUP; ++g) s[g] = 0.0f;
    if (lane < rows) {
        const uint32_t* krow = &ks[lane * AD_KROW];
#pragma unroll 4
        for (int j = 0; j < AD_D / 8; ++j) {
            const uint4 kk = *reinterpret_cast<const uint4*>(&krow[j * 4]);
            float kf[8];
            kf[0] = bf16_bits_to_f32(kk.x & 0xffffu); kf[1] = bf16_bits_to_f32(kk.x >> 16);
            kf[2] = bf16_bits_to_f32(kk.y & 0xffffu); kf[3] = bf16_bits_to_f32(kk.y >> 16);
            kf[4] = bf16_bits_to_f32(kk.z & 0xffffu); kf[5] = bf16_bits_to_f32(kk.z >> 16);
            kf[6] = bf16_bits_to_f32(kk.w & 0xffffu); kf[7] = bf16_bits_to_f32(kk.w >> 16);
#pragma unroll
            for (int g = 0; g < GROUP; ++g) {
                const float4 qa = *reinterpret_cast<const float4*>(&qs[g][j * 8]);
                const float4 qb = *reinterpret_cast<const float4*>(&qs[g][j * 8 + 4]);
                float t = s[g];
                t = fmaf(qa.x, kf[0], t); t = fmaf(qa.y, kf[1], t);
                t = fmaf(qa.z, kf[2], t); t = fmaf(qa.w, kf[3], t);
                t = fmaf(qb.x, kf[4], t); t = fmaf(qb.y, kf[5], t);
                t = fmaf(qb.z, kf[6], t); t = fmaf(qb.w, kf[7], t);
                s[g] = t;
            }
        }
    }

    // 6. chunk-local softmax statistics
    float mg[GROUP], lg[GROUP];
#pragma unroll
    for (int g = 0; g < GROUP; ++g) {
        const float sv = lane < rows ? s[g] : -INFINITY;
        const float m = wave_max(sv);
        const float e = lane < rows ? expf(sv - m) : 0.0f;
        mg[g] = m;
        lg[g] = wave_sum(e);
        ps[lane][g] = e;
    }
    __syncthreads();

    // 7. P.V: lane <-> dims (2*lane, 2*lane+1)
    float o0[GROUP], o1[GROUP];
#pragma unroll
    for (int g = 0; g < GROUP; ++g) o0[g] = o1[g] = 0.0f;
    for (int p = 0; p < rows; ++p) {
        const uint32_t vv = vs[p * (AD_D / 2) + lane];
        const float v0 = bf16_bits_to_f32(vv & 0xffffu);
        const float v1 = bf16_bits_to_f32(vv >> 16);
#pragma unroll
        for (int g = 0; g < GROUP; ++g) {
            const float pr = ps[p][g];
            o0[g] = fmaf(pr, v0, o0[g]);
            o1[g] = fmaf(pr, v1, o1[g]);
        }
    }

    // 8. publish the partial
    const size_t cbase = ((size_t)kvh * a.max_chunks + c) * GROUP;
#pragma unroll
    for (int g = 0; g < GROUP; ++g) {
        *reinterpret_cast<float2*>(&a.part_o[(cbase + g) * AD_D + 2 * lane]) = make_float2(o0[g], o1[g]);
        if (lane == 0) *reinterpret_cast<float2*>(&a.part_ml[(cbase + g) * 2]) = make_float2(mg[g], lg[g]);
    }
    __threadfence();
    uint32_t ticket = 0;
    if (lane == 0) ticket = atomicAdd(&a.tickets[kvh], 1u);
    ticket = (uint32_t)__shfl((int)ticket, 0, 64);
    if (ticket != (uint32_t)(n_chunks - 1)) return;
    __threadfence();

    // 9. last block of this kv head: log-sum-exp merge of all chunks
    const size_t hbase = (size_t)kvh * a.max_chunks * GROUP;
#pragma unroll
    for (int g = 0; g < GROUP; ++g) {
        float M = -INFINITY;
        for (int cc = 0; cc < n_chunks; ++cc) M = fmaxf(M, __builtin_nontemporal_load(&a.part_ml[(hbase + (size_t)cc * GROUP + g) * 2]));
        float lsum = 0.0f, acc0 = 0.0f, acc1 = 0.0f;
        for (int cc = 0; cc < n_chunks; ++cc) {
            const size_t idx = hbase + (size_t)cc * GROUP + g;
            const float m = __builtin_nontemporal_load(&a.part_ml[idx * 2]);
            const float l = __builtin_nontemporal_load(&a.part_ml[idx * 2 + 1]);
            const float f = expf(m - M);
            lsum = fmaf(f, l, lsum);
            const float2 ov = load_nt_f2(&a.part_o[idx * AD_D + 2 * lane]);
            acc0 = fmaf(f, ov.x, acc0);
            acc1 = fmaf(f, ov.y, acc1);
        }
        const float inv = 1.0f / lsum;
        const int h = kvh * GROUP + g;
        reinterpret_cast<uint32_t*>(a.out)[(h * AD_D) / 2 + lane] = pack_bf16x2(acc0 * inv, acc1 * inv);
    }
    if (lane == 0) a.tickets[kvh] = 0u;
}

}  // namespace t2h

using namespace t2h;

static uint32_t ad_max_chunks(uint32_t s_cap) { return (s_cap + AD_CH - 1) / AD_CH; }

static size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

extern "C" size_t t2h_attn_decode_workspace_bytes(uint32_t nh, uint32_t nk, uint32_t d, uint32_t s_cap) {
    if (nk == 0 || nh % nk != 0 || d != AD_D) return 0;
    const size_t group = nh / nk;
    const size_t mc = ad_max_chunks(s_cap);
    return align256(nk * sizeof(uint32_t)) + align256(nk * mc * group * 2 * sizeof(float)) +
           align256(nk * mc * group * d * sizeof(float));
}

extern "C" int t2h_attn_decode(const float* q, const float* k_new, const float* v_new, const float* q_norm_w,
                               const float* k_norm_w, float eps, float theta, void* k_cache, void* v_cache,
                               void* out, uint32_t nh, uint32_t nk, uint32_t d, uint32_t s_cap,
                               const int32_t* cache_position, void* workspace, size_t workspace_bytes,
                               void* stream) {
    if (!q || !k_new || !v_new || !k_cache || !v_cache || !out || !cache_position || !workspace) return T2H_ERR_NULL;
    if (d != AD_D) return T2H_ERR_UNSUPPORTED;
    if (nk == 0 || nh == 0 || nh % nk != 0 || s_cap == 0) return T2H_ERR_SHAPE;
    if ((q_norm_w == nullptr) != (k_norm_w == nullptr)) return T2H_ERR_ARG;
    const uint32_t group = nh / nk;
    if (workspace_bytes < t2h_attn_decode_workspace_bytes(nh, nk, d, s_cap)) return T2H_ERR_WORKSPACE;
    const uint32_t mc = ad_max_chunks(s_cap);
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
    a.tickets = reinterpret_cast<uint32_t*>(ws);
    ws += align256(nk * sizeof(uint32_t));
    a.part_ml = reinterpret_cast<float*>(ws);
    ws += align256((size_t)nk * mc * group * 2 * sizeof(float));
    a.part_o = reinterpret_cast<float*>(ws);
    a.nk = nk;
    a.s_cap = s_cap;
    a.max_chunks = mc;
    a.theta = theta;
    a.eps = eps;
    a.scale = 1.0f / sqrtf((float)d);
    const dim3 grid(mc, nk), block(64);
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    switch (group) {
        case 1: hipLaunchKernelGGL(attn_decode_kernel<1>, grid, block, 0, s, a); break;
        case 2: hipLaunchKernelGGL(attn_decode_kernel<2>, grid, block, 0, s, a); break;
        case 4: hipLaunchKernelGGL(attn_decode_kernel<4>, grid, block, 0, s, a); break;
        case 8: hipLaunchKernelGGL(attn_decode_kernel<8>, grid, block, 0, s, a); break;
        default: return T2H_ERR_UNSUPPORTED;
    }
    T2H_LAUNCH_CHECK();
    return T2H_OK;
}
