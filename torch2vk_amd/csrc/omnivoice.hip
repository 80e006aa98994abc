// OmniVoice's masked-generation token loop:
//   t2h_omnivoice_input_embed_q8_0   OMNIVOICE_INPUT_EMBED_Q8_0_F32
//   t2h_omnivoice_cfg_score          OMNIVOICE_CFG_SCORE_F32
//   t2h_omnivoice_token_update_topk  OMNIVOICE_TOKEN_UPDATE_TOPK_F32
// (src/models/quantized_omnivoice/shaders/omnivoice_*.py, driven from
// src/models/quantized_omnivoice/run.py:76-115).  Q8_0 rows: 34-byte blocks of
// an fp16 scale and 32 int8 values.
#include <cfloat>

#include "common.h"

namespace t2h {

__device__ __forceinline__ float ov_q8_0(const uint8_t* rows, size_t row_bytes, uint32_t row, uint32_t h) {
    const uint8_t* b = rows + (size_t)row * row_bytes + (size_t)(h >> 5) * 34;
    const float d = f16_bits_to_f32((uint32_t)b[0] | ((uint32_t)b[1] << 8));
    return d * (float)(int8_t)b[2 + (h & 31u)];
}

// hidden[b, s, h] = sum_c audio[c * V + ids[b, c, s]][h] where audio_mask[b, s],
// else text[ids[b, 0, s]][h]; a token outside its table contributes 0.
__global__ __launch_bounds__(256) void ov_input_embed_kernel(const uint8_t* __restrict__ text_w,
                                                             const uint8_t* __restrict__ audio_w,
                                                             const int64_t* __restrict__ ids,
                                                             const uint32_t* __restrict__ audio_mask,
                                                             float* __restrict__ out, uint32_t bsz, uint32_t c_books,
                                                             uint32_t s_len, uint32_t hdim, uint32_t vocab,
                                                             uint32_t n_text) {
    const uint64_t idx = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (uint64_t)bsz * s_len * hdim) return;
    const uint32_t h = (uint32_t)(idx % hdim);
    const uint64_t bs = idx / hdim;
    const uint32_t s = (uint32_t)(bs % s_len);
    const uint32_t b = (uint32_t)(bs / s_len);
    const size_t row_bytes = (size_t)(hdim / 32) * 34;
    float v = 0.0f;
    if (audio_mask[(uint64_t)b * s_len + s] != 0u) {
        for (uint32_t c = 0; c < c_books; ++c) {
            const int64_t tok = ids[((uint64_t)b * c_books + c) * s_len + s];
            if (tok >= 0 && tok < (int64_t)vocab) v += ov_q8_0(audio_w, row_bytes, c * vocab + (uint32_t)tok, h);
        }
    } else {
        const int64_t tok = ids[((uint64_t)b * c_books) * s_len + s];
        if (tok >= 0 && tok < (int64_t)n_text) v = ov_q8_0(text_w, row_bytes, (uint32_t)tok, h);
    }
    out[idx] = v;
}

// The hash and the Gumbel draw of OMNIVOICE_CFG_SCORE_F32 (a 32-bit integer
// mixer with the lowbias32 constants), kept exactly so that the same seed and
// step give the same noise.
__device__ __forceinline__ uint32_t ov_hash(uint32_t x) {
    x ^= x >> 16;
    x *= 0x7feb352du;
    x ^= x >> 15;
    x *= 0x846ca68bu;
    x ^= x >> 16;
    return x;
}

__device__ __forceinline__ float ov_gumbel(uint32_t seed, uint32_t step, uint32_t flat) {
    const uint32_t x = seed ^ (step * 0x9e3779b9u) ^ (flat * 0x85ebca6bu);
    float u = ((float)(ov_hash(x) & 0x00ffffffu) + 0.5f) * (1.0f / 16777216.0f);
    u = fminf(fmaxf(u, 1.0e-7f), 1.0f - 1.0e-7f);
    return -logf(-logf(u));
}

struct OvCfgArgs {
    const float* logits;      // [2, S, C * V]: batch 0 conditional, batch 1 unconditional
    const int64_t* tokens;    // [C * T]
    int64_t* cand_tokens;     // [C * T]
    float* cand_scores;       // [C * T]
    uint32_t s_len, c_books, t_len, vocab;
    float guidance, layer_penalty, temperature;
    uint32_t step, seed;
    int64_t mask_id;
};

__device__ __forceinline__ void ov_better(float& s, uint32_t& t, float s2, uint32_t t2) {
    if (s2 > s || (s2 == s && t2 < t)) {
        s = s2;
        t = t2;
    }
}

// One wave per (codebook c, target t): log-softmax of the conditional row
// (position S - T + t) and the unconditional row (position t) over codebook c's
// V logits, guided = c_lp + g (c_lp - u_lp), the best non-mask token (ties to the
// lowest id), its guided log-probability minus c * layer_penalty, optional
// Gumbel noise, and -FLT_MAX where the position is already decided.
__global__ __launch_bounds__(256) void ov_cfg_score_kernel(const OvCfgArgs a) {
    const uint32_t lane = threadIdx.x & 63;
    const uint64_t flat = (uint64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (flat >= (uint64_t)a.c_books * a.t_len) return;
    const uint32_t c = (uint32_t)(flat / a.t_len), t = (uint32_t)(flat % a.t_len);
    const size_t row = (size_t)a.c_books * a.vocab;
    const float* cl = a.logits + (size_t)(a.s_len - a.t_len + t) * row + (size_t)c * a.vocab;
    const float* ul = a.logits + (size_t)(a.s_len + t) * row + (size_t)c * a.vocab;
    float cm = -FLT_MAX, um = -FLT_MAX;
    for (uint32_t v = lane; v < a.vocab; v += 64) {
        cm = fmaxf(cm, cl[v]);
        um = fmaxf(um, ul[v]);
    }
    cm = wave_max(cm);
    um = wave_max(um);
    float cs = 0.0f, us = 0.0f;
    for (uint32_t v = lane; v < a.vocab; v += 64) {
        cs += expf(cl[v] - cm);
        us += expf(ul[v] - um);
    }
    const float c_norm = cm + logf(wave_sum(cs)), u_norm = um + logf(wave_sum(us));
    auto guided = [&](uint32_t v) {
        const float clp = cl[v] - c_norm, ulp = ul[v] - u_norm;
        return clp + a.guidance * (clp - ulp);
    };
    float gm = -FLT_MAX, best = -FLT_MAX;
    uint32_t best_tok = 0xffffffffu;
    for (uint32_t v = lane; v < a.vocab; v += 64) {
        const float g = guided(v);
        gm = fmaxf(gm, g);
        if ((int64_t)v != a.mask_id) ov_better(best, best_tok, g, v);
    }
    gm = wave_max(gm);
    float gs = 0.0f;
    for (uint32_t v = lane; v < a.vocab; v += 64) gs += expf(guided(v) - gm);
    gs = wave_sum(gs);
    for (int off = 32; off >= 1; off >>= 1) {
        const float s2 = __shfl_xor(best, off);
        const uint32_t t2 = __shfl_xor(best_tok, off);
        ov_better(best, best_tok, s2, t2);
    }
    if (lane != 0) return;
    float conf = best - gm - logf(gs);
    conf -= (float)c * a.layer_penalty;
    if (a.temperature > 0.0f) conf = conf / a.temperature + ov_gumbel(a.seed, a.step, (uint32_t)flat);
    if (a.tokens[flat] != a.mask_id) conf = -FLT_MAX;
    a.cand_tokens[flat] = (int64_t)best_tok;
    a.cand_scores[flat] = conf;
}

// Position i is unmasked when fewer than min(unmask_count, C T) positions rank
// above it (score descending, index ascending); its token goes to tokens[i] and
// to both copies of the sequence: conditional [0, c, S - T + t], unconditional [1, c, t].
__global__ __launch_bounds__(256) void ov_topk_kernel(const int64_t* __restrict__ cand_tokens,
                                                      const float* __restrict__ cand_scores,
                                                      int64_t* __restrict__ tokens, int64_t* __restrict__ ids,
                                                      uint32_t c_books, uint32_t t_len, uint32_t s_len,
                                                      uint32_t unmask_count) {
    const uint32_t total = c_books * t_len;
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= total) return;
    const uint32_t limit = min(unmask_count, total);
    const float s = cand_scores[i];
    uint32_t rank = 0;
    for (uint32_t j = 0; j < total; ++j) {
        const float o = cand_scores[j];
        rank += (o > s || (o == s && j < i)) ? 1u : 0u;
    }
    if (rank >= limit) return;
    const uint32_t c = i / t_len, t = i - c * t_len;
    const int64_t tok = cand_tokens[i];
    tokens[i] = tok;
    ids[((uint64_t)0 * c_books + c) * s_len + (s_len - t_len + t)] = tok;
    ids[((uint64_t)1 * c_books + c) * s_len + t] = tok;
}

}  // namespace t2h

using namespace t2h;

static inline uint32_t ov_grid(uint64_t threads, uint32_t per_block) {
    return (uint32_t)((threads + per_block - 1) / per_block);
}

extern "C" int t2h_omnivoice_input_embed_q8_0(const void* text_w, uint32_t n_text, const void* audio_w,
                                              const int64_t* ids, const uint32_t* audio_mask, float* out,
                                              uint32_t batch, uint32_t codebooks, uint32_t seq, uint32_t hidden,
                                              uint32_t vocab, void* stream) {
    if (!text_w || !audio_w || !ids || !audio_mask || !out) return T2H_ERR_NULL;
    if (hidden == 0 || hidden % 32 != 0 || codebooks == 0) return T2H_ERR_SHAPE;
    const uint64_t n = (uint64_t)batch * seq * hidden;
    if (n == 0) return T2H_OK;
    if (n / 256 >= 0x7fffffffu || (uint64_t)codebooks * vocab > 0xffffffffu) return T2H_ERR_SHAPE;
    hipLaunchKernelGGL(ov_input_embed_kernel, dim3(ov_grid(n, 256)), dim3(256), 0,
                       reinterpret_cast<hipStream_t>(stream), reinterpret_cast<const uint8_t*>(text_w),
                       reinterpret_cast<const uint8_t*>(audio_w), ids, audio_mask, out, batch, codebooks, seq, hidden,
                       vocab, n_text);
    T2H_LAUNCH_CHECK();
    return T2H_OK;
}

extern "C" int t2h_omnivoice_cfg_score(const float* logits, const int64_t* tokens, int64_t* cand_tokens,
                                       float* cand_scores, uint32_t seq, uint32_t codebooks, uint32_t targets,
                                       uint32_t vocab, float guidance, float layer_penalty, float temperature,
                                       uint32_t step, uint32_t seed, int64_t mask_id, void* stream) {
    if (!logits || !tokens || !cand_tokens || !cand_scores) return T2H_ERR_NULL;
    if (vocab == 0 || targets > seq) return T2H_ERR_SHAPE;
    const uint64_t n = (uint64_t)codebooks * targets;
    if (n == 0) return T2H_OK;
    if (n / 4 >= 0x7fffffffu) return T2H_ERR_SHAPE;
    OvCfgArgs a;
    a.logits = logits;
    a.tokens = tokens;
    a.cand_tokens = cand_tokens;
    a.cand_scores = cand_scores;
    a.s_len = seq;
    a.c_books = codebooks;
    a.t_len = targets;
    a.vocab = vocab;
    a.guidance = guidance;
    a.layer_penalty = layer_penalty;
    a.temperature = temperature;
    a.step = step;
    a.seed = seed;
    a.mask_id = mask_id;
    hipLaunchKernelGGL(ov_cfg_score_kernel, dim3(ov_grid(n, 4)), dim3(256), 0, reinterpret_cast<hipStream_t>(stream),
                       a);
    T2H_LAUNCH_CHECK();
    return T2H_OK;
}

extern "C" int t2h_omnivoice_token_update_topk(const int64_t* cand_tokens, const float* cand_scores, int64_t* tokens,
                                               int64_t* batch_input_ids, uint32_t codebooks, uint32_t targets,
                                               uint32_t seq, uint32_t unmask_count, void* stream) {
    if (!cand_tokens || !cand_scores || !tokens || !batch_input_ids) return T2H_ERR_NULL;
    if (targets > seq) return T2H_ERR_SHAPE;
    const uint64_t n = (uint64_t)codebooks * targets;
    if (n == 0) return T2H_OK;
    if (n > 0xffffffffu) return T2H_ERR_SHAPE;
    hipLaunchKernelGGL(ov_topk_kernel, dim3(ov_grid(n, 256)), dim3(256), 0, reinterpret_cast<hipStream_t>(stream),
                       cand_tokens, cand_scores, tokens, batch_input_ids, codebooks, targets, seq, unmask_count);
    T2H_LAUNCH_CHECK();
    return T2H_OK;
}
