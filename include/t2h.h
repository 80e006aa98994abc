/*
 * libt2h - MI355X (gfx950) kernels for torch2vk's quantized Qwen3 hot path.
 *
 * C ABI: plain device pointers, sizes and a hipStream_t passed as void*.
 * Every entry point enqueues work on the caller's stream and returns a status
 * (0 = ok).  Nothing here allocates device memory or synchronises the host:
 * scratch space is a caller-provided workspace of a queried size, and dynamic
 * scalars (cache position, token index) are device pointers, so a caller can
 * capture any sequence of calls into a HIP graph and replay it.
 *
 * Packed weight formats are the GGUF blocks the reference's kernels read
 * (src/torch2vk/checkpoints/gguf.py:79-95, src/torch2vk/vulkan/types.py:64-82):
 *   Q4_K: 144 B / 256 values, Q6_K: 210 B / 256 values, Q8_0: 34 B / 32 values,
 * row-major, one row per output feature.  Activations are bf16 (reference:
 * fp16, src/torch2vk/export/dtype_policy.py:23-36); accumulation is fp32.
 *
 * Citations are to files under the reference tree taowen/torch2vk.
 */
#ifndef T2H_H
#define T2H_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------ status ---- */
/* The reference raises ValueError/TypeError before a launch
 * (src/torch2vk/runtime/dispatcher.py:35-53); these are the same checks. */
enum {
    T2H_OK = 0,
    T2H_ERR_NULL = 1,        /* a required pointer is null */
    T2H_ERR_SHAPE = 2,       /* shape violates the contract (e.g. K % 256 != 0) */
    T2H_ERR_DTYPE = 3,       /* unsupported dtype combination */
    T2H_ERR_UNSUPPORTED = 4, /* valid but not built (e.g. head_dim != 128) */
    T2H_ERR_ARG = 5,         /* other invalid argument */
    T2H_ERR_WORKSPACE = 6,   /* workspace smaller than the queried size */
    T2H_ERR_ALIGN = 7,       /* pointer not 16-byte aligned */
    T2H_ERR_HIP_BASE = 1000  /* 1000 + hipError_t of a failed launch */
};

enum { T2H_DTYPE_F32 = 0, T2H_DTYPE_BF16 = 1 };
enum { T2H_WTYPE_Q4_K = 12, T2H_WTYPE_Q6_K = 14, T2H_WTYPE_Q8_0 = 8, T2H_WTYPE_BF16 = 30 }; /* GGUF type ids,
                                                                                          gguf.py:19-53 */

int t2h_abi_version(void);
const char* t2h_status_string(int status);

/* --------------------------------------------------------- quantizers --- */
/* fp32 [rows, k] -> packed GGUF rows, bit-identical to the reference GLSL
 * restated with IEEE RNE rounding and no fma contraction. */
/* replaces quantize_q4_k_vulkan / GGUF_QUANTIZE_Q4_K_F32, src/torch2vk/quantize/vulkan.py:39-50,188-419 */
int t2h_quantize_q4_k(const float* x, uint32_t rows, uint32_t k, void* out, void* stream);
/* replaces quantize_q6_k_vulkan / GGUF_QUANTIZE_Q6_K_F32, src/torch2vk/quantize/vulkan.py:53-66,422-636 */
int t2h_quantize_q6_k(const float* x, uint32_t rows, uint32_t k, void* out, void* stream);
/* replaces quantize_q8_0_vulkan / GGUF_QUANTIZE_Q8_0_F32, src/torch2vk/quantize/vulkan.py:25-36,91-185
 * (k must already be padded to a multiple of 32, as gguf.py:125-127 declares) */
int t2h_quantize_q8_0(const float* x, uint32_t rows, uint32_t k, void* out, void* stream);
/* packed rows -> fp32 [rows, k]; the reference decoders' value formula
 * (src/models/quantized_qwen3/shaders/embedding_q4_k_f32.py:97-110 and the K6/K7 decoders) */
int t2h_dequantize(int wtype, const void* w, uint32_t rows, uint32_t k, float* out, void* stream);

/* ------------------------------------------------------ decode GEMVs ---- */
/* y[m, n] = x[m, k] . deq(W[n, k])^T (+ residual[m, n]); x bf16, out fp32 or bf16.
 * replaces LINEAR_NOBIAS_Q4_K_MATVEC_F32 (src/models/optimized_qwen3/shaders/linear_nobias_q4_k_matvec_f32.py:26-197)
 * and, with residual != NULL (fp32 out), LINEAR_NOBIAS_Q4_K_MATVEC_ADD_F32
 * (src/models/optimized_qwen3/shaders/linear_nobias_q4_k_matvec_add_f32.py:23-100).  residual may alias y. */
int t2h_q4k_matvec(const void* x, const void* w, void* y, int out_dtype, const float* residual, uint32_t m,
                   uint32_t k, uint32_t n, void* stream);

/* Up to 3 weights sharing one x read: Q|K|V or gate|up.  With norm_w != NULL,
 * x is the fp32 residual stream and RMSNorm(x)*norm_w is fused as a prologue.
 * replaces LINEAR_NOBIAS_Q4_K_QKV_MATVEC_F32 (src/models/optimized_qwen3/shaders/linear_nobias_q4_k_qkv_matvec_f32.py:22-430),
 * LINEAR_NOBIAS_Q4_K_QK_MATVEC_F32 (.../linear_nobias_q4_k_qk_matvec_f32.py:22-315) and, fused in front,
 * RMS_NORM_MUL_F16_F32 (.../rms_norm_mul_f16_f32.py:22-115). */
int t2h_q4k_matvec_multi(const void* x, const float* norm_w, float eps, uint32_t n_parts, const void* const* w,
                         void* const* y, const uint32_t* n, uint32_t k, int out_dtype, void* stream);

/* act[n] = silu(g) * u with g|u = RMSNorm(h)*norm_w . deq(W_gate|W_up)^T; act bf16.
 * replaces RMS_NORM_MUL_F16_F32 + LINEAR_NOBIAS_Q4_K_QK_MATVEC_F32 + SWIGLU_F16
 * (src/models/optimized_qwen3/dispatch/decode_layer.py:107-121). */
int t2h_q4k_rmsnorm_swiglu_matvec(const float* h, const float* norm_w, float eps, const void* w_gate,
                                  const void* w_up, void* act_out, uint32_t k, uint32_t n, void* stream);

/* LM head GEMV fused with a per-block argmax; logits are never materialised.
 * x: bf16 normed hidden (norm_w == NULL) or fp32 residual stream with the
 * final RMSNorm fused (norm_w != NULL).  Writes num_partials (score, token)
 * pairs; ties go to the lower token id.
 * replaces LM_HEAD_Q6_K_ARGMAX_PARTIAL_F16 (src/torch2vk/export/shaders/lm_head_q6_k_argmax_partial_f16.py:24-209)
 * for Q4_K weights, plus run_decode_norm in front (src/models/optimized_qwen3/dispatch/decode_norm.py). */
int t2h_q4k_lm_head_argmax_partial(const void* x, const float* norm_w, float eps, const void* w, uint32_t k,
                                   uint32_t n, float* partial_scores, uint32_t* partial_tokens,
                                   uint32_t num_partials, void* stream);

/* t2h_q4k_lm_head_argmax_partial with the final RMSNorm fused, for n_seq (1..4) sequences that decode
 * together: the head's rows are read once, and sequence i's fp32 residual stream h[i] gives its own
 * num_partials (score, token) pairs in partial_scores[i] / partial_tokens[i], bit-identical to the
 * single-sequence call.  k is 1024 or 4096 (other k: T2H_ERR_UNSUPPORTED).
 * replaces one LM_HEAD_Q6_K_ARGMAX_PARTIAL_F16 dispatch per sequence (src/models/optimized_qwen3/run.py:116-122,
 * _run_lm_head_select, called once per decode step at run.py:162) for the sequences of a batched decode. */
int t2h_q4k_lm_head_argmax_partial_seqs(uint32_t n_seq, const float* const* h, const float* norm_w, float eps,
                                        const void* w, uint32_t k, uint32_t n, float* const* partial_scores,
                                        uint32_t* const* partial_tokens, uint32_t num_partials, void* stream);

/* Q6_K GEMV: y[m, n] = x[m, k] . deq(W)^T (+ residual), x bf16, k % 256 == 0,
 * k <= 12288 (longer rows: T2H_ERR_UNSUPPORTED).
 * replaces LINEAR_NOBIAS_Q6_K_MATVEC_F32 (src/models/quantized_qwen3/shaders/linear_nobias_q6_k_matvec_f32.py:20-193)
 * and, with residual, LINEAR_NOBIAS_Q6_K_MATVEC_ADD_F32
 * (src/models/optimized_qwen3/shaders/linear_nobias_q6_k_matvec_add_f32.py:23-100). */
int t2h_q6k_matvec(const void* x, const void* w, void* y, int out_dtype, const float* residual, uint32_t m,
                   uint32_t k, uint32_t n, void* stream);

/* Q6_K GEMV of RMSNorm(h)*norm_w for one token (h fp32 residual stream):
 * the v_proj of the Q4_K_M "more bits" layers.
 * replaces RMS_NORM_MUL_F16_F32 + the Q6_K part of LINEAR_NOBIAS_Q4_QK_Q6_V_MATVEC_F32
 * (src/models/optimized_qwen3/shaders/linear_nobias_q4_qk_q6_v_matvec_f32.py:103-160). */
int t2h_q6k_rmsnorm_matvec(const float* h, const float* norm_w, float eps, const void* w, void* y, int out_dtype,
                           uint32_t k, uint32_t n, void* stream);

/* Q8_0 GEMV: y[m, n] = x[m, k] . deq(W)^T (+ residual), x bf16 (converted to
 * fp16 in-kernel, the reference's activation type), k % 32 == 0, k <= 12288.
 * replaces LINEAR_NOBIAS_Q8_0_MATVEC_F32 (src/models/quantized_qwen3/shaders/linear_nobias_q8_0_matvec_f32.py:24-119). */
int t2h_q8_0_matvec(const void* x, const void* w, void* y, int out_dtype, const float* residual, uint32_t m,
                    uint32_t k, uint32_t n, void* stream);

/* 1 when t2h_q4k_matvec / t2h_q6k_matvec / t2h_q8_0_matvec (wtype T2H_WTYPE_*) are built for rows of k
 * values and n output rows, else 0 (those calls would return T2H_ERR_UNSUPPORTED or T2H_ERR_SHAPE).
 * The reference's matvec shaders take any K and N; a caller routes the other shapes to the GEMM.
 * serves the kernel choice of make_linear_nobias_q4_k_m_variant
 * (src/torch2vk/export/shaders/linear_nobias_quantized.py:47-80). */
int t2h_matvec_supported(int wtype, uint32_t k, uint32_t n);

/* Q6_K LM head + per-block argmax, as t2h_q4k_lm_head_argmax_partial.
 * replaces LM_HEAD_Q6_K_ARGMAX_PARTIAL_F16 (src/torch2vk/export/shaders/lm_head_q6_k_argmax_partial_f16.py:24-209). */
int t2h_q6k_lm_head_argmax_partial(const void* x, const float* norm_w, float eps, const void* w, uint32_t k,
                                   uint32_t n, float* partial_scores, uint32_t* partial_tokens,
                                   uint32_t num_partials, void* stream);

/* Grid caps of the Q4_K GEMV launches, in blocks (tuning knob, process-wide):
 * max_blocks for plain bf16 x (default 256), max_blocks_norm for the fused
 * RMSNorm prologue (default 256; 0 = same as max_blocks).  Each wave gets
 * ceil(units / (blocks * waves)) row units.  No reference counterpart: the
 * reference fixes its grids in the shader variants. */
int t2h_set_gemv_max_blocks(uint32_t max_blocks, uint32_t max_blocks_norm);

/* ------------------------------------------------------ prefill GEMMs --- */
/* y[m, n] = x[m, k] . deq(W[n, k])^T (+ residual) on the matrix cores: x bf16
 * (16-byte aligned), W dequantised to bf16 tiles in LDS, fp32 accumulation,
 * out fp32 or bf16 (fp32 with residual, which may alias y).  Any m and n; k % 64 == 0.
 * replaces LINEAR_NOBIAS_Q8_0_F32 (src/models/quantized_qwen3/shaders/linear_nobias_q8_0_f32.py:24-209). */
int t2h_q8_0_gemm(const void* x, const void* w, void* y, int out_dtype, const float* residual, uint32_t m,
                  uint32_t k, uint32_t n, void* stream);
/* replaces LINEAR_NOBIAS_Q4_K_F32 (src/models/quantized_qwen3/shaders/linear_nobias_q4_k_f32.py:26-296) and
 * LLAMA_MATMUL_Q4_K_F32_{M,L} (src/models/optimized_qwen3/shaders/llama_matmul_q4_k_f32.py:32-141); k % 256 == 0. */
int t2h_q4k_gemm(const void* x, const void* w, void* y, int out_dtype, const float* residual, uint32_t m,
                 uint32_t k, uint32_t n, void* stream);
/* y bf16 [m, n_ff] = silu(x . deq(W_gate)^T) * (x . deq(W_up)^T): the prefill MLP's gate and up GEMMs and
 * the SwiGLU in one launch (each wave's tile columns pair 32 gate rows with the 32 up rows of the same
 * features).  wtype T2H_WTYPE_Q8_0 / Q4_K / Q6_K / BF16, both weights [n_ff, k]; k % 64 == 0 (% 256 for the
 * K types).  replaces LLAMA_MATMUL_Q4_K_F32_{M,L} x 2 + SWIGLU_F32 (src/models/optimized_qwen3/dispatch/
 * text_layer.py; src/models/optimized_qwen3/shaders/swiglu_f32.py). */
int t2h_gemm_swiglu(int wtype, const void* x, const void* w_gate, const void* w_up, void* y, uint32_t m, uint32_t k,
                    uint32_t n_ff, void* stream);
/* Split-K form of the prefill GEMMs above, for grids too small to fill the GPU (a few hundred rows, as in a
 * short prompt or a 512-token prefill chunk): K is cut into `splits` equal parts of whole 64-wide stages, each
 * part's fp32 products go to partials (t2h_gemm_splitk_bytes(m, n, splits, swiglu) bytes, 16-B aligned),
 * then a second kernel sums the parts in order and applies the epilogue: bias,
 * act, and fp32 (+ residual, which may alias y) or bf16 output.  w_up non-null selects the SwiGLU form (w the
 * gate rows, n = n_ff features, y bf16 [m, n_ff]; no bias, act or residual).  wtype Q8_0 / Q4_K / Q6_K / BF16;
 * w_k as t2h_q8_0_linear (= k for the K types and for SwiGLU); 1 <= splits <= min(k / 64, 64).  The results
 * equal the one-pass GEMM's up to the order of the fp32 sum.  No counterpart of its own in the reference: it
 * is the same LINEAR_NOBIAS_*_F32 / LLAMA_MATMUL_*_F32 products (see the entries above), scheduled for small
 * M. */
size_t t2h_gemm_splitk_bytes(uint32_t m, uint32_t n, uint32_t splits, int swiglu);
int t2h_gemm_splitk(int wtype, const void* x, const void* w, const void* w_up, const float* bias, int act, void* y,
                    int out_dtype, const float* residual, uint32_t m, uint32_t k, uint32_t n, uint32_t w_k,
                    uint32_t splits, void* partials, size_t partials_bytes, void* stream);
/* The same GEMM over bf16 weight rows (GGUF BF16, 16-byte aligned): the tiles are copied into LDS instead of
 * dequantised.  Any m and n; k % 64 == 0.  replaces LINEAR_NOBIAS_BF16W_F32
 * (src/models/exported_qwen3_asr/shaders/linear_nobias_bf16w_f32.py, whose activations are fp16 where these are
 * bf16), and runs the prefill GEMMs over weights dequantised once by t2h_dequantize_bf16. */
int t2h_bf16_gemm(const void* x, const void* w, void* y, int out_dtype, const float* residual, uint32_t m,
                  uint32_t k, uint32_t n, void* stream);
/* t2h_q8_0_linear's epilogues (bias, GELU, residual) over bf16 weight rows [n, k]: the encoder linears at
 * large M over weights dequantised once (t2h_dequantize_bf16), bit-identical to t2h_q8_0_linear on the packed
 * rows when they hold k values.  replaces LINEAR_BIAS_BF16W_BF16B_F32
 * (src/models/exported_qwen3_asr/shaders/linear_bias_bf16w_bf16b_f32.py, bf16 bias there, fp32 here). */
int t2h_bf16_linear(const void* x, const void* w, const float* bias, int act, void* y, int out_dtype,
                    const float* residual, uint32_t m, uint32_t k, uint32_t n, void* stream);
/* out bf16 [rows, k] (16-byte aligned) = the bf16 values the GEMMs above dequantise W's rows to in LDS (wtype
 * Q8_0 / Q4_K / Q6_K; k % 64 == 0, % 256 for the K types), so that t2h_bf16_gemm / t2h_gemm_swiglu(BF16) over
 * out give bit-identical results to the quantized GEMM on W.  For large prefills, where the quantized GEMM
 * would dequantise every weight tile once per 256 rows of x: dequantised once here, each tile is only copied.
 * No reference counterpart (the reference dequantises inside every GEMM workgroup,
 * src/models/quantized_qwen3/shaders/linear_nobias_q8_0_f32.py:24-209). */
int t2h_dequantize_bf16(int wtype, const void* w, uint32_t rows, uint32_t k, void* out, void* stream);
/* replaces LLAMA_MATMUL_Q6_K_F32_{M,L} (src/models/optimized_qwen3/shaders/llama_matmul_q6_k_f32.py:27-141):
 * the Q6_K v/down weights of the Q4_K_M more-bits layers; k % 256 == 0, W 2-byte aligned. */
int t2h_q6k_gemm(const void* x, const void* w, void* y, int out_dtype, const float* residual, uint32_t m,
                 uint32_t k, uint32_t n, void* stream);
/* y[m, n] = act(x[m, k] . deq(W[n, w_k])^T + bias) (+ residual), W Q8_0 rows of w_k / 32 blocks, w_k <= k,
 * w_k % 32 == 0, k % 64 == 0 (columns of x past w_k multiply zeros; keep them finite).  bias fp32 [n] or
 * NULL; act 0 = none, 1 = GELU (erf by Abramowitz-Stegun 7.1.26, as the reference's GELU); out fp32 or bf16
 * (fp32 with residual, which may alias y).
 * replaces LINEAR_BIAS_Q8_0W_F32B_F32 (src/models/quantized_qwen3_asr/shaders/linear_bias_q8_0w_f32b_f32.py:27-213)
 * and, after t2h_im2col, CONV2D_Q8_0W_F32B_F16{,_2,_3} (shaders/conv2d_q8_0w_f32b_f16.py:25-136); the GELU that
 * follows each of them in the audio tower (dispatch/audio_encoder.py:27-63) is fused here. */
int t2h_q8_0_linear(const void* x, const void* w, const float* bias, int act, void* y, int out_dtype,
                    const float* residual, uint32_t m, uint32_t k, uint32_t n, uint32_t w_k, void* stream);

/* ---------------------------------------------------- token selection --- */
/* replaces QWEN3_TOKEN_SELECT_REDUCE_CHUNKS_F32 + QWEN3_TOKEN_SELECT_REDUCE_F32
 * (src/torch2vk/export/shaders/qwen3_token_select_reduce_f32.py:22-241): one pass over g partials. */
int t2h_token_select(const float* scores, const uint32_t* tokens, uint32_t g, const int64_t* eos, uint32_t n_eos,
                     int64_t* next_token, uint32_t* done, void* stream);

/* replaces QWEN3_TOKEN_STORE_EOS_F32 (src/models/optimized_qwen3/shaders/qwen3_token_store_eos_f32.py:21-140).
 * token_index_ptr (device, nullable) overrides token_index; advance (device,
 * nullable) is incremented once per call for graph-replayed loops. */
int t2h_token_store(const int64_t* next_token, const uint32_t* done, int64_t* generated, uint32_t g,
                    uint32_t* length, uint32_t* stopped, uint32_t stop_on_eos, const uint32_t* token_index_ptr,
                    uint32_t token_index, int32_t* advance, void* stream);

/* Select and store fused into one launch (the same two reference shaders):
 * next_token/done as t2h_token_select; the token is appended at
 * generated[*length] (if < gen_cap and not stopped), *length += 1, *stopped set
 * on EOS when stop_on_eos; *advance (nullable) += 1 on every call. */
int t2h_token_select_store(const float* scores, const uint32_t* tokens, uint32_t g, const int64_t* eos,
                           uint32_t n_eos, int64_t* next_token, uint32_t* done, int64_t* generated, uint32_t gen_cap,
                           uint32_t* length, uint32_t* stopped, uint32_t stop_on_eos, int32_t* advance, void* stream);

/* t2h_token_select_store for n_seq (1..4) sequences that decode together, in one launch: sequence i's
 * partials, token, flags, generated ids, counters and (nullable) advance counter are element i of each
 * pointer array; done[i] and advance[i] may be null; g, eos, gen_cap and stop_on_eos are shared.  Each
 * sequence's result equals its own t2h_token_select_store call.
 * replaces one QWEN3_TOKEN_SELECT_REDUCE_F32 + QWEN3_TOKEN_STORE_EOS_F32 pair per sequence
 * (src/models/optimized_qwen3/run.py:123-139 and the token store of its decode loop) for a batched decode. */
int t2h_token_select_store_seqs(uint32_t n_seq, const float* const* scores, const uint32_t* const* tokens, uint32_t g,
                                const int64_t* eos, uint32_t n_eos, int64_t* const* next_token, uint32_t* const* done,
                                int64_t* const* generated, uint32_t gen_cap, uint32_t* const* length,
                                uint32_t* const* stopped, uint32_t stop_on_eos, int32_t* const* advance, void* stream);

/* ------------------------------------------------- decode attention ---- */
/* Split-K flash decoding over a bf16 token-major cache [s_cap, nk, d] (d = 128).
 * q [nh, d], k_new/v_new [nk, d] fp32 projections.  With q_norm_w/k_norm_w,
 * per-head RMSNorm is applied; with theta > 0, rotate-half RoPE at
 * *cache_position.  The new K/V row is written at *cache_position (if
 * < s_cap) and attention covers positions 0..min(*cache_position, s_cap-1).
 * out bf16 [nh, d].  workspace: t2h_attn_decode_workspace_bytes() bytes of
 * per-chunk partials (no initialisation needed); calls sharing one workspace
 * must not overlap in time.  Two launches: the split-K pass and a
 * log-sum-exp merge.
 * replaces RMS_NORM_ROPE_TRANSPOSE_F16 x2 (src/models/optimized_qwen3/shaders/rms_norm_rope_transpose_f16.py:22-145),
 * ROPE_TABLE_F32 (src/torch2vk/runtime/rope_table.py:32-122) and
 * SDPA_DECODE_CACHE_WRITE_F32 (src/models/optimized_qwen3/shaders/sdpa_decode_cache_write_f32.py:22-170). */
size_t t2h_attn_decode_workspace_bytes(uint32_t nh, uint32_t nk, uint32_t d, uint32_t s_cap);
int t2h_attn_decode(const float* q, const float* k_new, const float* v_new, const float* q_norm_w,
                    const float* k_norm_w, float eps, float theta, void* k_cache, void* v_cache, void* out,
                    uint32_t nh, uint32_t nk, uint32_t d, uint32_t s_cap, const int32_t* cache_position,
                    void* workspace, size_t workspace_bytes, void* stream);

/* --------------------------------------------- persistent decode layers --- */
/* Every decoder layer of one Qwen3 decode token in one launch: for each layer,
 * RMSNorm + Q|K|V GEMV, q/k-norm + RoPE + KV-cache write + split-K attention
 * and its merge, o_proj + residual, RMSNorm + gate|up + SwiGLU, down +
 * residual, on h (fp32 [hidden], updated in place), at *cache_position.
 * Same arithmetic as the per-op entry points; 256 resident blocks (one per CU)
 * pass the activations between phases as epoch-tagged words and poll for them,
 * with no grid barrier (no host sync, graph-capturable).  Calls on one
 * workspace must not overlap in time.
 * Built for the Qwen3-8B shape (hidden 4096, mlp 12288, 32/8 heads), the Qwen3-1.7B shape (hidden 2048,
 * mlp 6144, 16/8 heads) and the Qwen3-0.6B shape (hidden 1024, mlp 3072, 16/8 heads), d 128, Q4_K weights with v and down each Q4_K or Q6_K per layer (the uniform
 * and Q4_K_M policies), bf16 KV caches [s_cap, 8, 128] with s_cap <= 8192, n_layers <= 64 (otherwise
 * T2H_ERR_UNSUPPORTED; so is a GPU that cannot hold 256 blocks).
 * layer_table: device int64 [n_layers][14]: pointers in the order
 *   wq, wk, wv, wo, w_gate, w_up, w_down, input_norm, post_norm, q_norm, k_norm, k_cache, v_cache,
 * then the layer's weight types: bit 0 set = wv is Q6_K, bit 1 set = w_down is Q6_K.  wq and wk must be one
 * allocation of q_dim + kv_dim stacked rows (wk = wq + q_dim rows); a Q4_K wv must continue it (wv = wk +
 * kv_dim rows), a Q6_K wv is an allocation of its own.
 * workspace: t2h_qwen3_decode_layers_workspace_bytes() bytes, 256-B aligned,
 * zero-filled once before its first use (it holds a launch counter that later
 * calls advance).  *status (device) is set to 0x80000000 | layer << 8 | phase
 * (phase 1..7: qkv, attention q, attention k/v, merge, o, gate/up, down) if a
 * wait for another block's output timed out, which means the result is
 * invalid; it is never cleared by the library.
 * replaces run_decode_layer for every layer (src/models/optimized_qwen3/dispatch/decode_layer.py:60-136;
 * decode step src/models/optimized_qwen3/run.py:142-172). */
size_t t2h_qwen3_decode_layers_workspace_bytes(uint32_t hidden, uint32_t mlp, uint32_t nh, uint32_t nk, uint32_t d);
int t2h_qwen3_decode_layers(const uint64_t* layer_table, uint32_t n_layers, uint32_t hidden, uint32_t mlp, uint32_t nh,
                            uint32_t nk, uint32_t d, uint32_t s_cap, float* h, const int32_t* cache_position, float eps,
                            float theta, void* workspace, size_t workspace_bytes, uint32_t* status, void* stream);
/* t2h_qwen3_decode_layers without a workspace argument, for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid allocation).  No counterpart in the
 * reference.  The workspace is a file-scope device array of 1.5 MiB per GPU (held until the process ends, zero at
 * load), large enough for both built shapes; a shape whose workspace would exceed it returns T2H_ERR_WORKSPACE.
 * The first call on a GPU looks up that GPU's copy of the array (hipGetSymbolAddress, no allocation).  Every call
 * on one GPU shares the array and its launch counter: calls that overlap in time on one GPU race, and no call may
 * overlap a launch of t2h_qwen3_decode_layers on the same GPU that uses this array as its workspace.  Results are
 * bit-identical to t2h_qwen3_decode_layers on the same inputs. */
int t2h_qwen3_decode_layers_noalloc(const uint64_t* layer_table, uint32_t n_layers, uint32_t hidden, uint32_t mlp,
                                    uint32_t nh, uint32_t nk, uint32_t d, uint32_t s_cap, float* h,
                                    const int32_t* cache_position, float eps, float theta, uint32_t* status,
                                    void* stream);
/* n_seq independent decode sequences in one launch, each with its own layer table (its own KV caches; the
 * weights may be shared), h, *cache_position, workspace (t2h_qwen3_decode_layers_workspace_bytes(), distinct per
 * sequence) and *status, as t2h_qwen3_decode_layers; all share n_layers, the shape, s_cap, eps and theta.  The
 * host arrays hold n_seq device pointers each.  n_seq = 1 is t2h_qwen3_decode_layers; n_seq = 4 is built for
 * the Qwen3-0.6B shape with s_cap <= 2048: the 256 blocks split into 4 groups of 64, one per sequence, each
 * streaming its own copy of the weights (at this shape the hand-offs, not HBM, bound a launch, so four
 * sequences take little longer than one).  No counterpart in the reference, which decodes one sequence at a
 * time (run_decode_layer, src/models/optimized_qwen3/dispatch/decode_layer.py:60-136, per sequence). */
int t2h_qwen3_decode_layers_seqs(uint32_t n_seq, const uint64_t* const* layer_tables, uint32_t n_layers,
                                 uint32_t hidden, uint32_t mlp, uint32_t nh, uint32_t nk, uint32_t d, uint32_t s_cap,
                                 float* const* hs, const int32_t* const* cache_positions, float eps, float theta,
                                 void* const* workspaces, size_t workspace_bytes, uint32_t* const* statuses,
                                 void* stream);
/* The same launch with a phase timeline: trace (device, 8-B aligned, t2h_qwen3_decode_layers_trace_bytes()
 * bytes) receives, per layer, phase (qkv, attention, merge, o, gate/up, down) and block (256), 8 uint64 slots:
 * the 100 MHz real-time clock at the phase's start, when its input is in hand, after its first reduced unit
 * (attention: its softmax), at its end, then the polls its first wave made for the input.  A separate kernel
 * instantiation with the stamps compiled in; a diagnostic with no counterpart in the reference, which profiles
 * its dispatches with SQTT traces instead (src/torch2vk/runtime/profile.py). */
size_t t2h_qwen3_decode_layers_trace_bytes(uint32_t n_layers);
int t2h_qwen3_decode_layers_traced(const uint64_t* layer_table, uint32_t n_layers, uint32_t hidden, uint32_t mlp,
                                   uint32_t nh, uint32_t nk, uint32_t d, uint32_t s_cap, float* h,
                                   const int32_t* cache_position, float eps, float theta, void* workspace,
                                   size_t workspace_bytes, uint32_t* status, uint64_t* trace, size_t trace_bytes,
                                   void* stream);
/* t2h_qwen3_decode_layers_seqs with the same timeline: one trace buffer for the launch, indexed by the grid's
 * block, so with n_seq = 4 sequence i's stamps are blocks 64 i .. 64 i + 63. */
int t2h_qwen3_decode_layers_seqs_traced(uint32_t n_seq, const uint64_t* const* layer_tables, uint32_t n_layers,
                                        uint32_t hidden, uint32_t mlp, uint32_t nh, uint32_t nk, uint32_t d,
                                        uint32_t s_cap, float* const* hs, const int32_t* const* cache_positions,
                                        float eps, float theta, void* const* workspaces, size_t workspace_bytes,
                                        uint32_t* const* statuses, uint64_t* trace, size_t trace_bytes, void* stream);

/* -------------------------------------------------- prefill attention --- */
/* out = softmax(q.k^T * scale + mask) . v on the matrix cores (bf16 in, fp32
 * scores and accumulation, bf16 out).  q, out: [batch, t_len, nh, d] and k, v:
 * [batch, s_len, nk, d] addressed through strides (in elements, all >= 0):
 *   strides[0..2]  q   (batch, token, head)     strides[3..5]  k
 *   strides[6..8]  v                             strides[9..11] out
 *   strides[12..13] mask (batch, query row); the key index is contiguous.
 * The head dimension is contiguous (d = 64 or 128).  GQA: kv head = h / (nh/nk).
 * causal != 0: query t sees keys <= t + causal_offset.  mask: additive fp32
 * (natural-log units) or NULL.  scale <= 0 means 1/sqrt(d).  Alignment: q, k
 * 16 B with their strides multiples of 8; v, out 8 B with strides multiples of 4.
 * A query that sees no key gets zeros.
 * replaces LLAMA_FLASH_ATTN_F32_F16_F16 (src/models/optimized_qwen3/shaders/llama_flash_attn_f32_f16_f16.py:35-175),
 * SDPA_CAUSAL_F32 (src/models/quantized_qwen3/shaders/sdpa_causal_f32.py:22-142) and
 * SDPA_MASKED_F32 (src/models/optimized_qwen3_asr/shaders/sdpa_masked_f32.py). */
int t2h_flash_attn_prefill(const void* q, const void* k, const void* v, void* out, const float* mask, uint32_t batch,
                           uint32_t nh, uint32_t nk, uint32_t t_len, uint32_t s_len, uint32_t d,
                           const int64_t* strides, int causal, int32_t causal_offset, float scale, void* stream);
/* Class of every block of 128 queries x 64 keys of an additive fp32 mask [mask_batch][t_len][s_len] (element
 * strides m_sb, m_st; keys contiguous): 1 if every entry is <= -FLT_MAX/2 (all masked), 2 if every entry is 0,
 * else 0; tiles uint8 [mask_batch][ceil(t_len/128)][ceil(s_len/64)].
 * replaces FA_MASK_OPT_F16 (src/models/optimized_qwen3/shaders/fa_mask_opt_f16.py:20-60; its rule, on this
 * kernel's block shape). */
int t2h_fa_mask_tiles(const float* mask, uint32_t mask_batch, uint32_t t_len, uint32_t s_len, int64_t m_sb,
                      int64_t m_st, uint8_t* tiles, void* stream);
/* t2h_flash_attn_prefill with the mask's tile classes (t2h_fa_mask_tiles over the same mask; one row of tiles
 * for every batch when strides[12] is 0): all-masked tiles are skipped, all-zero tiles are not read.  The
 * result equals t2h_flash_attn_prefill's, except that a query whose every key is masked gets zeros.
 * replaces LLAMA_FLASH_ATTN_F32_F16_F16 driven with its mask-opt buffer
 * (src/models/optimized_qwen3/run.py:406,437). */
int t2h_flash_attn_prefill_tiles(const void* q, const void* k, const void* v, void* out, const float* mask,
                                 const uint8_t* mask_tiles, uint32_t batch, uint32_t nh, uint32_t nk, uint32_t t_len,
                                 uint32_t s_len, uint32_t d, const int64_t* strides, int causal, int32_t causal_offset,
                                 float scale, void* stream);
/* Self-attention within segments: token t attends to the keys of its own segment [cu[i], cu[i+1]),
 * cu_seqlens int32 [n_seg + 1] on the device, ascending, cu[0] = 0, cu[n_seg] = t_len (a token outside
 * [cu[0], cu[n_seg]) gets zeros).  Same tensors and strides[0..11] as t2h_flash_attn_prefill with
 * s_len = t_len.  Equals SDPA_MASKED_F32 with the Qwen3-ASR block-diagonal window mask
 * (src/models/quantized_qwen3_asr/pytorch_modules.py:95-114, shaders/sdpa_masked_f32.py) without reading a
 * mask: key tiles outside a block's segments are skipped. */
/* Prefill chunk prologue: for tokens t < n at positions start + t, per-head RMSNorm (q_norm_w / k_norm_w,
 * both or neither) and rotate-half RoPE (theta <= 0: none) of q [n, q_row] and k [n, k_row] (fp32, head h at
 * columns 128 h); q -> q_out bf16 [n, nh, 128], k and v [n, v_row] -> bf16 cache rows [s_cap, nk, 128] at the
 * tokens' positions (start + n <= s_cap).  d must be 128.  Same per-token math as t2h_attn_decode's prologue.
 * replaces RMS_NORM_ROPE_TOKEN_F32{,_TO_F16} (src/models/optimized_qwen3/shaders/rms_norm_rope_token_f32.py:22-99)
 * and TOKEN_MAJOR_{KV,VALUE}_CACHE_WRITE_* (shaders/token_major_kv_cache_write_f16_pair.py:20-103). */
int t2h_qk_norm_rope_cache(const float* q, uint64_t q_row, const float* k, uint64_t k_row, const float* v,
                           uint64_t v_row, const float* q_norm_w, const float* k_norm_w, float eps, float theta,
                           int32_t start, uint32_t n, uint32_t nh, uint32_t nk, uint32_t d, void* q_out,
                           void* k_cache, void* v_cache, uint32_t s_cap, void* stream);
/* The same prologue for n_seq sequences of n tokens each, in one launch (a batched prefill): q, k, v and q_out
 * have n_seq * n rows (sequence s at rows s n ..), each sequence's tokens are at positions start + t, and the
 * caches hold n_seq consecutive [s_cap, nk, 128] caches, one per sequence.  n_seq = 1 is
 * t2h_qk_norm_rope_cache.  Replaces the same shaders, run per sequence of a batch. */
int t2h_qk_norm_rope_cache_seqs(const float* q, uint64_t q_row, const float* k, uint64_t k_row, const float* v,
                                uint64_t v_row, const float* q_norm_w, const float* k_norm_w, float eps, float theta,
                                int32_t start, uint32_t n, uint32_t n_seq, uint32_t nh, uint32_t nk, uint32_t d,
                                void* q_out, void* k_cache, void* v_cache, uint32_t s_cap, void* stream);
int t2h_flash_attn_segments(const void* q, const void* k, const void* v, void* out, const int32_t* cu_seqlens,
                            uint32_t n_seg, uint32_t batch, uint32_t nh, uint32_t nk, uint32_t t_len, uint32_t d,
                            const int64_t* strides, float scale, void* stream);

/* ------------------------------------------------------ small ops ------ */
/* replaces EMBEDDING_Q4_K_F32 (src/models/quantized_qwen3/shaders/embedding_q4_k_f32.py:62-121); out fp32 [n_ids, dim] */
int t2h_embedding_q4_k(const void* w, uint64_t vocab, const int64_t* ids, uint32_t n_ids, uint32_t dim, float* out,
                       void* stream);
/* One token of each of n_seq (1..4) sequences: out[i] (fp32 [dim], 16-byte aligned) = row ids[i][0] of the
 * Q4_K embedding, as t2h_embedding_q4_k.  replaces one EMBEDDING_Q4_K_F32 dispatch per sequence
 * (src/models/quantized_qwen3/shaders/embedding_q4_k_f32.py:62-121, run_decode_embed) for a batched decode. */
int t2h_embedding_q4_k_seqs(uint32_t n_seq, const void* w, uint64_t vocab, const int64_t* const* ids, uint32_t dim,
                            float* const* out, void* stream);
/* replaces RMS_NORM_MUL_F16_F32 / RMS_NORM_MUL_F32 (src/models/optimized_qwen3/shaders/rms_norm_mul_f16_f32.py:22-115) */
int t2h_rms_norm(const void* x, int x_dtype, const float* w, void* out, int out_dtype, uint32_t rows, uint32_t h,
                 float eps, void* stream);
/* replaces SWIGLU_F16 / SWIGLU_F32 (src/models/optimized_qwen3/shaders/swiglu_f16.py:20-81); out bf16 */
int t2h_swiglu(const void* gate, const void* up, int in_dtype, void* out, uint64_t n, void* stream);

/* ------------------------------------------- Qwen3-ASR audio tower ----- */
/* out[(b, oh, ow), (c, fh, fw)] = x[b, c, oh*stride_h + fh - pad_h, ow*stride_w + fw - pad_w] (0 outside),
 * bf16 rows of out_cols >= channels*kh*kw (the rest zero-filled); x fp32 or bf16 addressed by element strides
 * (b, c, h, w).  The conv2d front-end's patch gather (CONV2D_Q8_0W_F32B_F16, src/models/quantized_qwen3_asr/
 * shaders/conv2d_q8_0w_f32b_f16.py:114-136) and, with an (F x 1) kernel, the flatten + transpose before conv_out
 * (pytorch_modules.py:463-466). */
int t2h_im2col(const void* x, int x_dtype, const int64_t* x_strides, uint32_t batch, uint32_t channels,
               uint32_t in_h, uint32_t in_w, uint32_t kh, uint32_t kw, uint32_t stride_h, uint32_t stride_w,
               uint32_t pad_h, uint32_t pad_w, uint32_t out_h, uint32_t out_w, void* out, uint32_t out_cols,
               void* stream);
/* conv1d taps of x [B, C, L] (fp32 or bf16, any element strides x_strides[3] = b, c, l): bf16 out
 * [B * out_len, out_cols], row b * out_len + t, column c * K + k = x[b, c, t * stride + k * dilation - pad]
 * (zero outside the input); columns past C * K are zero.  With a Q8_0 GEMM over [Co, C * K] weight rows
 * (t2h_q8_0_linear) this is CONV1D_Q8_0W_F32B_F32 (src/models/quantized_omnivoice/shaders/
 * conv1d_q8_0w_f32b_f32.py: conv_input_value, q8_0_value_prepared), stride, padding and dilation included. */
int t2h_im2col_1d(const void* x, int x_dtype, const int64_t* x_strides, uint32_t batch, uint32_t channels,
                  uint32_t length, uint32_t k, uint32_t stride, uint32_t pad, uint32_t dilation, uint32_t out_len,
                  void* out, uint32_t out_cols, void* stream);
/* Snake activation over channels-last fp32 rows [rows, C]: out = x + sin(alpha_c x)^2 / (alpha_c + eps).
 * Replaces ADD_SCALAR + RECIPROCAL_F32 + AUDIO_DECODE_MUL_BROADCAST + SIN_F32 + POW_SCALAR_F16 + ADD
 * (src/models/quantized_omnivoice/dispatch/audio_decode.py:151-161; eps 1e-9, add_scalar.py:43). */
int t2h_snake(const float* x, const float* alpha, float* out, uint64_t rows, uint32_t channels, float eps,
              void* stream);
/* Transposed conv1d with Q8_0 weights: x fp32 [B, Ci, L_in] (any element strides x_strides[3] = b, c, l),
 * w the reference's Q8_0 rows [Ci, ceil(Co * K / 32) * 34 bytes] (element co * K + k of row ci), bias fp32
 * [Co] or NULL; out fp32 [B, L_out, Co] contiguous, L_out = (L_in - 1) * stride - 2 pad + K + output padding,
 * the output padding in [0, stride) (the reference's blocks write stride * L_in outputs: kernel 2 stride, pad
 * ceil(stride / 2), output padding stride % 2; the extra positions take the taps that reach them).
 * y[b, t, co] = bias[co] + sum over ci and the taps k with t + pad - k = i * stride, 0 <= i < L_in, of
 * W[ci, co * K + k] x[b, ci, i].  Replaces CONV_TRANSPOSE1D_Q8_0W_F32B_F32
 * (src/models/quantized_omnivoice/shaders/conv_transpose1d_q8_0w_f32b_f32.py). */
int t2h_conv_transpose1d_q8_0(const float* x, const int64_t* x_strides, const void* w, const float* bias, float* out,
                              uint32_t batch, uint32_t ci, uint32_t li, uint32_t co, uint32_t kh, uint32_t stride,
                              uint32_t pad, uint32_t lo, void* stream);

/* ----------------------------------------------- OmniVoice token loop --- */
/* hidden fp32 [B, S, H] = sum over c < C of audio_w row (c * V + ids[b, c, s]) where audio_mask[b, s] != 0,
 * else text_w row ids[b, 0, s]; Q8_0 rows of H values (H % 32 == 0); ids int64 [B, C, S], audio_mask uint32
 * [B, S]; a token outside its table contributes 0.  Replaces OMNIVOICE_INPUT_EMBED_Q8_0_F32
 * (src/models/quantized_omnivoice/shaders/omnivoice_input_embed_q8_0_f32.py). */
int t2h_omnivoice_input_embed_q8_0(const void* text_w, uint32_t n_text, const void* audio_w, const int64_t* ids,
                                   const uint32_t* audio_mask, float* out, uint32_t batch, uint32_t codebooks,
                                   uint32_t seq, uint32_t hidden, uint32_t vocab, void* stream);
/* Per (codebook c, target t) of C x T: log-softmax over codebook c's V logits of the conditional row
 * (logits[0, S - T + t]) and the unconditional row (logits[1, t]) of fp32 logits [2, S, C * V]; guided =
 * c + guidance (c - u); the best token other than mask_id (ties to the lowest id) and its guided
 * log-probability minus c * layer_penalty, divided by temperature plus Gumbel noise (the reference's hash
 * of seed, step and position) when temperature > 0, and -FLT_MAX where tokens[c T + t] != mask_id.
 * Replaces OMNIVOICE_CFG_SCORE_F32 (src/models/quantized_omnivoice/shaders/omnivoice_cfg_score_f32.py). */
int t2h_omnivoice_cfg_score(const float* logits, const int64_t* tokens, int64_t* cand_tokens, float* cand_scores,
                            uint32_t seq, uint32_t codebooks, uint32_t targets, uint32_t vocab, float guidance,
                            float layer_penalty, float temperature, uint32_t step, uint32_t seed, int64_t mask_id,
                            void* stream);
/* Unmask the min(unmask_count, C T) best candidates (score descending, index ascending): tokens[i] and
 * batch_input_ids int64 [2, C, S] at [0, c, S - T + t] and [1, c, t] take cand_tokens[i].  Replaces
 * OMNIVOICE_TOKEN_UPDATE_TOPK_F32 (src/models/quantized_omnivoice/shaders/omnivoice_token_update_topk_f32.py). */
int t2h_omnivoice_token_update_topk(const int64_t* cand_tokens, const float* cand_scores, int64_t* tokens,
                                    int64_t* batch_input_ids, uint32_t codebooks, uint32_t targets, uint32_t seq,
                                    uint32_t unmask_count, void* stream);
/* out = (x - mean) / sqrt(var + eps) * w + b per row (biased variance, two passes); x, out fp32 or bf16,
 * cols % 4 == 0, 16-B aligned.  replaces LAYER_NORM_F32W_F32B_F32
 * (src/models/quantized_qwen3_asr/shaders/layer_norm_f32w_f32b_f32.py:20-105). */
int t2h_layer_norm(const void* x, int x_dtype, const float* w, const float* b, void* out, int out_dtype,
                   uint32_t rows, uint32_t cols, float eps, void* stream);
/* out = x * (1 + erf(x / sqrt 2)) / 2; n % 4 == 0.  replaces GELU_F32 (src/models/quantized_qwen3_asr/shaders/
 * gelu_f32.py:22-82) where it is not fused into t2h_q8_0_linear. */
int t2h_gelu(const void* x, int x_dtype, void* out, int out_dtype, uint64_t n, void* stream);
/* out[i] = src[idx[i]] for rows of row_bytes (% 4); an index outside [0, src_rows) gives a zero row.
 * replaces INDEX_SELECT_F32 (src/models/quantized_qwen3_asr/shaders/index_select_f32_c6680f8d95.py). */
int t2h_index_select_rows(const void* src, uint64_t src_rows, uint32_t row_bytes, const int64_t* idx, uint32_t n,
                          void* out, void* stream);
/* dst[idx[i]] = src[i] for rows of row_bytes (% 4); an index outside [0, dst_rows) is skipped.
 * replaces INDEX_COPY_F32 (src/models/quantized_qwen3_asr/shaders/index_copy_f32_7ba4f1ff13.py; the audio
 * injection, dispatch/audio_inject.py:11-13). */
int t2h_index_copy_rows(void* dst, uint64_t dst_rows, uint32_t row_bytes, const int64_t* idx, uint32_t n,
                        const void* src, void* stream);
/* out fp32 [n_ids, dim] = deq(W[ids]) for Q8_0 rows of dim / 32 blocks; an id outside [0, vocab) gives zeros.
 * replaces EMBEDDING_Q8_0_F32 (src/models/quantized_qwen3_asr/shaders/embedding_q8_0_f32.py:25-97). */
int t2h_embedding_q8_0(const void* w, uint64_t vocab, const int64_t* ids, uint32_t n_ids, uint32_t dim, float* out,
                       void* stream);

/* ------------------------------------ the reference's unfused operators --- */
/* cos / sin fp32 [B, T, D] of positions start + t (start from *start_position_ptr when it is not NULL, else
 * start_position): inv_freq(d) = theta^(-2 (d mod D/2) / D), values times attention_scaling.  The factors the
 * fused kernels compute in registers (rope.h), bit for bit.  replaces ROPE_TABLE_F32
 * (src/torch2vk/runtime/rope_table.py:32-122). */
int t2h_rope_table(float* cos_out, float* sin_out, uint32_t b, uint32_t t, uint32_t d, float theta,
                   uint32_t start_position, const int32_t* start_position_ptr, float attention_scaling, void* stream);
/* Per-head RMSNorm over D = 128 (weight fp32 [D], eps) then rotate-half RoPE from a table:
 * out[d] = n[d] cos[d] - n[d + 64] sin[d], out[d + 64] = n[d + 64] cos[d + 64] + n[d] sin[d + 64], per row
 * (b, t, g) of x [B, T, G, D] (fp32 or bf16) with the table row (b, t) of cos / sin fp32 [B, T, D]; out fp32 or
 * bf16 [B, T, G, D], or [B, G, T, D] with transpose_out.  replaces RMS_NORM_ROPE_TRANSPOSE_F16
 * (src/models/optimized_qwen3/shaders/rms_norm_rope_transpose_f16.py:22-145) and RMS_NORM_ROPE_TOKEN_F32 /
 * _TO_F16 (src/models/optimized_qwen3/shaders/rms_norm_rope_token_f32.py:22-99). */
int t2h_rms_norm_rope(const void* x, int x_dtype, const float* weight, const float* cos_table,
                      const float* sin_table, void* out, int out_dtype, uint32_t b, uint32_t t, uint32_t g, uint32_t d,
                      int transpose_out, float eps, void* stream);
/* Rows src [B, T, H, D] (fp32 or bf16) into n_caches (1..3) token-major bf16 caches [B, s_caps[c], H, D] at
 * positions[t] (int64 [T]; a position outside a cache writes nothing there).  replaces
 * TOKEN_MAJOR_KV_CACHE_WRITE_F16_PAIR / _TRIPLE and TOKEN_MAJOR_VALUE_CACHE_WRITE_F32_TO_F16_PAIR / _TRIPLE
 * (src/models/optimized_qwen3/shaders/token_major_kv_cache_write_f16_pair.py:20-103). */
int t2h_kv_cache_write(const void* src, int src_dtype, const int64_t* positions, uint32_t n_caches,
                       void* const* caches, const uint32_t* s_caps, uint32_t b, uint32_t t, uint32_t h, uint32_t d,
                       void* stream);
/* The best (score, token) of each chunk of 1024 of g partials (ties to the lower token id): chunk_scores /
 * chunk_tokens [ceil(g / 1024)].  replaces QWEN3_TOKEN_SELECT_REDUCE_CHUNKS_F32
 * (src/torch2vk/export/shaders/qwen3_token_select_reduce_f32.py:22-120). */
int t2h_token_select_chunks(const float* scores, const uint32_t* tokens, uint32_t g, float* chunk_scores,
                            uint32_t* chunk_tokens, void* stream);
/* out = x + y over n elements of dtype (fp32, or bf16 with an fp32 sum rounded once); out may alias x or y.
 * replaces ADD_F32_PREFILL (src/models/optimized_qwen3/shaders/add_f32_prefill.py:20-60) and ADD_F32_36
 * (src/models/optimized_qwen3/shaders/add_f32_36.py:22-80). */
int t2h_add(const void* x, const void* y, void* out, int dtype, uint64_t n, void* stream);
/* out [B, 1, H] (fp32 or bf16) = row S - 1 of each batch of x fp32 [B, S, H].  replaces
 * SLICE_LAST_TOKEN_F32_TO_F16 (src/models/optimized_qwen3/shaders/slice_last_token_f32_to_f16.py:19-60). */
int t2h_slice_last_token(const float* x, void* out, int out_dtype, uint32_t b, uint32_t s, uint32_t h, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* T2H_H */
