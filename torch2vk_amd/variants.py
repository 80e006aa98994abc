"""The reference's decode and prefill operators under their own names, as ``ShaderVariant`` objects.

Each variant keeps the reference shader's name, field names, symbolic shapes and weight layouts
(src/models/optimized_qwen3/shaders/*.py, src/models/quantized_qwen3/shaders/*.py,
src/torch2vk/export/shaders/linear_nobias_quantized.py), is called as ``VARIANT(rt, **tensors)`` and, once
``RuntimeSession.dispatch`` has checked the call, runs one libt2h entry point.  Where this library's kernel does
more than the reference's (an RMSNorm prologue, q/k norm and RoPE fused into attention), the variant runs it in
the reference's narrower meaning.  Activations are bf16 (the reference's fp16), the residual stream fp32.
"""

from __future__ import annotations

import torch

from torch2vk_amd import kernels
from torch2vk_amd.runtime import (
    Q4_K_WORDS,
    Q6_K_HALFWORDS,
    Q8_0_HALFWORDS,
    IOKind,
    PushConstantInput,
    RuntimeSession,
    ShaderContract,
    ShaderVariant,
    TensorContract,
    TensorFieldSpec,
    ceil_div,
    mul,
)

ACT = "bfloat16"
OUT = ("float32", "bfloat16")
F32 = "float32"

_LAYOUT_WTYPE = {Q4_K_WORDS: "q4_k", Q6_K_HALFWORDS: "q6_k", Q8_0_HALFWORDS: "q8_0"}


def _weight(name: str, rows: str, layout: str, k: str = "K") -> TensorFieldSpec:
    if layout == Q4_K_WORDS:
        c = TensorContract("uint32", (rows, mul(ceil_div(k, 256), 36)), layout)
    elif layout == Q6_K_HALFWORDS:
        c = TensorContract("uint16", (rows, mul(ceil_div(k, 256), 105)), layout)
    else:
        c = TensorContract("uint16", (rows, mul(ceil_div(k, 32), 17)), layout)
    return TensorFieldSpec(name, IOKind.INPUT, "weight", c)


def _f(name: str, io: IOKind, dtype, shape) -> TensorFieldSpec:
    return TensorFieldSpec(name, io, "input" if io is IOKind.INPUT else ("state" if io is IOKind.INOUT else "output"),
                           TensorContract(dtype, tuple(shape)))


def _bytes(w: torch.Tensor) -> torch.Tensor:
    """The GGUF rows of a word or halfword weight tensor, as the bytes the kernels read (no copy)."""
    return w.view(torch.uint8)


def _variant(name: str, class_name: str, fields, launch, push=()) -> ShaderVariant:
    return ShaderVariant(name=name, family="t2h", contract=ShaderContract(class_name, name, tuple(fields), tuple(push)),
                         launch=launch)


def _rows(sym, name: str, limit: int) -> int:
    m = sym["X0"] * sym["X1"]
    if m > limit:
        raise ValueError(f"{name} is a matrix-vector kernel for at most {limit} rows, got {m}")
    return m


# ------------------------------------------------------------------ GEMVs (M <= 8) --

def _matvec(name: str, class_name: str, layout: str, residual: bool) -> ShaderVariant:
    fields = [_f("x", IOKind.INPUT, ACT, ("X0", "X1", "K")), _weight("weight", "N", layout)]
    if residual:
        fields.append(_f("residual", IOKind.INPUT, F32, ("X0", "X1", "N")))
    fields.append(_f("output", IOKind.OUTPUT, F32 if residual else OUT, ("X0", "X1", "N")))

    def launch(rt: RuntimeSession, t, sym, push) -> None:
        _rows(sym, name, kernels.GEMV_MAX_ROWS)
        wtype = _LAYOUT_WTYPE[layout]
        res = t["residual"] if residual else None
        if not kernels.matvec_supported(wtype, sym["K"], sym["N"]):
            # a row length or row count the GEMVs are not built for: the same product on the GEMM
            kernels.gemm(t["x"], _bytes(t["weight"]), wtype, out=t["output"], residual=res)
        elif wtype == "q4_k":
            kernels.q4k_matvec(t["x"], _bytes(t["weight"]), out=t["output"], residual=res)
        else:
            kernels.qx_matvec(t["x"], _bytes(t["weight"]), wtype, out=t["output"], residual=res)

    return _variant(name, class_name, fields, launch)


# src/models/optimized_qwen3/shaders/linear_nobias_q4_k_matvec_f32.py:26-197
LINEAR_NOBIAS_Q4_K_MATVEC_F32 = _matvec("linear_nobias_q4_k_matvec_f32", "LinearNobiasQ4KMatvecProgram", Q4_K_WORDS,
                                        False)
# src/models/optimized_qwen3/shaders/linear_nobias_q4_k_matvec_add_f32.py:23-100
LINEAR_NOBIAS_Q4_K_MATVEC_ADD_F32 = _matvec("linear_nobias_q4_k_matvec_add_f32", "LinearNobiasQ4KMatvecAddProgram",
                                            Q4_K_WORDS, True)
# src/models/quantized_qwen3/shaders/linear_nobias_q6_k_matvec_f32.py:20-193
LINEAR_NOBIAS_Q6_K_MATVEC_F32 = _matvec("linear_nobias_q6_k_matvec_f32", "LinearNobiasQ6KMatvecProgram",
                                        Q6_K_HALFWORDS, False)
# src/models/optimized_qwen3/shaders/linear_nobias_q6_k_matvec_add_f32.py:23-100
LINEAR_NOBIAS_Q6_K_MATVEC_ADD_F32 = _matvec("linear_nobias_q6_k_matvec_add_f32", "LinearNobiasQ6KMatvecAddProgram",
                                            Q6_K_HALFWORDS, True)
# src/models/quantized_qwen3/shaders/linear_nobias_q8_0_matvec_f32.py:24-119
LINEAR_NOBIAS_Q8_0_MATVEC_F32 = _matvec("linear_nobias_q8_0_matvec_f32", "LinearNobiasQ8_0MatvecProgram",
                                        Q8_0_HALFWORDS, False)


def _multi(name: str, class_name: str, parts: tuple[tuple[str, str], ...]) -> ShaderVariant:
    """Several weights sharing one input row: ((prefix, layout), ...) with fields {prefix}_weight / {prefix}_output."""
    fields = [_f("x", IOKind.INPUT, ACT, ("X0", "X1", "K"))]
    for prefix, layout in parts:
        fields.append(_weight(f"{prefix}_weight", f"N{prefix.upper()}", layout))
    for prefix, _ in parts:
        fields.append(_f(f"{prefix}_output", IOKind.OUTPUT, OUT, ("X0", "X1", f"N{prefix.upper()}")))

    def launch(rt: RuntimeSession, t, sym, push) -> None:
        if _rows(sym, name, 1) != 1:
            raise ValueError(f"{name} takes one row")
        dtypes = {t[f"{p}_output"].dtype for p, _ in parts}
        if len(dtypes) != 1:
            raise TypeError(f"{name}: every output must have the same dtype")
        q4 = [p for p, layout in parts if layout == Q4_K_WORDS]
        x = t["x"].view(-1)
        kernels.q4k_matvec_multi(x, [_bytes(t[f"{p}_weight"]) for p in q4], [t[f"{p}_output"].view(-1) for p in q4])
        for p, layout in parts:
            if layout != Q4_K_WORDS:
                kernels.qx_matvec(x.view(1, -1), _bytes(t[f"{p}_weight"]), _LAYOUT_WTYPE[layout],
                                  out=t[f"{p}_output"])

    return _variant(name, class_name, fields, launch)


# src/models/optimized_qwen3/shaders/linear_nobias_q4_k_qkv_matvec_f32.py:22-430
LINEAR_NOBIAS_Q4_K_QKV_MATVEC_F32 = _multi("linear_nobias_q4_k_qkv_matvec_f32", "LinearNobiasQ4KQkvMatvecProgram",
                                           (("q", Q4_K_WORDS), ("k", Q4_K_WORDS), ("v", Q4_K_WORDS)))
# src/models/optimized_qwen3/shaders/linear_nobias_q4_k_qk_matvec_f32.py:22-315 (gate|up in the MLP)
LINEAR_NOBIAS_Q4_K_QK_MATVEC_F32 = _multi("linear_nobias_q4_k_qk_matvec_f32", "LinearNobiasQ4KQkMatvecProgram",
                                          (("q", Q4_K_WORDS), ("k", Q4_K_WORDS)))
# src/models/optimized_qwen3/shaders/linear_nobias_q4_qk_q6_v_matvec_f32.py:103-160
LINEAR_NOBIAS_Q4_QK_Q6_V_MATVEC_F32 = _multi("linear_nobias_q4_qk_q6_v_matvec_f32",
                                             "LinearNobiasQ4QkQ6VMatvecProgram",
                                             (("q", Q4_K_WORDS), ("k", Q4_K_WORDS), ("v", Q6_K_HALFWORDS)))


# --------------------------------------------------------- prefill GEMMs (M > 8) --

def _gemm(name: str, class_name: str, layout: str) -> ShaderVariant:
    fields = [_f("x", IOKind.INPUT, ACT, ("X0", "X1", "K")), _weight("weight", "N", layout),
              _f("output", IOKind.OUTPUT, OUT, ("X0", "X1", "N"))]

    def launch(rt: RuntimeSession, t, sym, push) -> None:
        kernels.gemm(t["x"], _bytes(t["weight"]), _LAYOUT_WTYPE[layout], out=t["output"])

    return _variant(name, class_name, fields, launch)


# src/models/quantized_qwen3/shaders/linear_nobias_q4_k_f32.py:26-296
LINEAR_NOBIAS_Q4_K_F32 = _gemm("linear_nobias_q4_k_f32", "LinearNobiasQ4KProgram", Q4_K_WORDS)
# src/models/quantized_qwen3/shaders/linear_nobias_q8_0_f32.py:24-209
LINEAR_NOBIAS_Q8_0_F32 = _gemm("linear_nobias_q8_0_f32", "LinearNobiasQ8_0Program", Q8_0_HALFWORDS)
# the Q6_K tile loader of src/models/optimized_qwen3/shaders/llama_matmul_q6_k_f32.py
LINEAR_NOBIAS_Q6_K_F32 = _gemm("linear_nobias_q6_k_f32", "LinearNobiasQ6KProgram", Q6_K_HALFWORDS)

_MATVEC = {Q4_K_WORDS: LINEAR_NOBIAS_Q4_K_MATVEC_F32, Q6_K_HALFWORDS: LINEAR_NOBIAS_Q6_K_MATVEC_F32,
           Q8_0_HALFWORDS: LINEAR_NOBIAS_Q8_0_MATVEC_F32}
_GEMM = {Q4_K_WORDS: LINEAR_NOBIAS_Q4_K_F32, Q6_K_HALFWORDS: LINEAR_NOBIAS_Q6_K_F32,
         Q8_0_HALFWORDS: LINEAR_NOBIAS_Q8_0_F32}


def linear_nobias_quantized_variant(m: int, layout: str) -> ShaderVariant:
    """The variant make_linear_nobias_q4_k_m_variant picks (src/torch2vk/export/shaders/linear_nobias_quantized.py:
    47-80): the matrix-vector kernel for M <= 8 rows, the matrix-core GEMM above, of the weight's layout."""
    return (_MATVEC if m <= kernels.GEMV_MAX_ROWS else _GEMM)[layout]


def run_linear_nobias_quantized(rt: RuntimeSession, *, x: torch.Tensor, weight: torch.Tensor,
                                output: torch.Tensor) -> None:
    """One linear of any GGUF weight type at any M: run_quantized_linear over the variants the rows select."""
    from torch2vk_amd.runtime import run_quantized_linear

    m = x.numel() // int(x.shape[-1])
    pick = _MATVEC if m <= kernels.GEMV_MAX_ROWS else _GEMM
    run_quantized_linear(rt, q4=pick[Q4_K_WORDS], q6=pick[Q6_K_HALFWORDS], q8=pick[Q8_0_HALFWORDS], x=x,
                         weight=weight, output=output)


# ------------------------------------------------------------ norm, SwiGLU, embed --

def _rms_launch(rt: RuntimeSession, t, sym, push) -> None:
    kernels.rms_norm(t["x"], t["weight"], out=t["output"])


# src/models/optimized_qwen3/shaders/rms_norm_mul_f16_f32.py:22-115 (eps 1e-6, fp32 reduction)
RMS_NORM_MUL_F16_F32 = _variant(
    "rms_norm_mul_f16_f32", "RmsNormMulProgram",
    [_f("x", IOKind.INPUT, OUT, ("X0", "X1", "H")), _f("weight", IOKind.INPUT, F32, ("H",)),
     _f("output", IOKind.OUTPUT, OUT, ("X0", "X1", "H"))], _rms_launch)


def _swiglu_launch(rt: RuntimeSession, t, sym, push) -> None:
    if t["up"].dtype != t["gate"].dtype:
        raise TypeError("swiglu_f16: gate and up must have the same dtype")
    kernels.swiglu(t["gate"], t["up"], out=t["output"])


# src/models/optimized_qwen3/shaders/swiglu_f16.py:20-81
SWIGLU_F16 = _variant(
    "swiglu_f16", "SwigluProgram",
    [_f("gate", IOKind.INPUT, OUT, ("X0", "X1", "N")), _f("up", IOKind.INPUT, OUT, ("X0", "X1", "N")),
     _f("output", IOKind.OUTPUT, ACT, ("X0", "X1", "N"))], _swiglu_launch)


def _embed_launch(rt: RuntimeSession, t, sym, push) -> None:
    kernels.embedding_q4_k(_bytes(t["weight"]), t["indices"].view(-1), sym["H"], out=t["output"].view(-1, sym["H"]))


# src/models/quantized_qwen3/shaders/embedding_q4_k_f32.py:62-121
EMBEDDING_Q4_K_F32 = _variant(
    "embedding_q4_k_f32", "EmbeddingQ4KProgram",
    [_weight("weight", "V", Q4_K_WORDS, "H"), _f("indices", IOKind.INPUT, "int64", ("B", "T")),
     _f("output", IOKind.OUTPUT, F32, ("B", "T", "H"))], _embed_launch)


# ------------------------------------------------------------------ decode attention --

def _position(rt: RuntimeSession, value) -> torch.Tensor:
    """cache_position as the device int32 the kernel reads (a Python int is written into a session buffer)."""
    if isinstance(value, torch.Tensor):
        return value.view(-1)
    buf = rt.workspace("cache_position", 4).view(torch.int32)
    buf.fill_(int(value))
    return buf


def _sdpa_decode(norm_rope: bool, theta: float, eps: float):
    def launch(rt: RuntimeSession, t, sym, push) -> None:
        if sym["B"] != 1 or sym["T"] != 1:
            raise ValueError("decode attention takes one sequence and one token (B = T = 1)")
        nh, nk, s, d = sym["NH"], sym["NK"], sym["S"], sym["D"]
        pos = int(push["cache_position"]) if not isinstance(push["cache_position"], torch.Tensor) else None
        if pos is not None and pos >= s:
            raise ValueError(f"cache_position {pos} outside the cache of {s} positions")
        ws = rt.workspace("attn_decode", kernels.attn_decode_workspace_bytes(nh, nk, d, s))
        kernels.attn_decode(t["q"].view(nh, d), t["new_k"].view(nk, d), t["new_v"].view(nk, d), t["k_cache"][0],
                            t["v_cache"][0], t["output"].view(-1), _position(rt, push["cache_position"]), ws,
                            q_norm_weight=t["q_norm_weight"] if norm_rope else None,
                            k_norm_weight=t["k_norm_weight"] if norm_rope else None,
                            theta=theta if norm_rope else 0.0, eps=eps)

    return launch


_SDPA_FIELDS = [
    _f("q", IOKind.INPUT, F32, ("B", "NH", "T", "D")),
    _f("new_k", IOKind.INPUT, F32, ("B", "NK", "T", "D")),
    _f("new_v", IOKind.INPUT, F32, ("B", "T", "NK", "D")),
    _f("k_cache", IOKind.INOUT, ACT, ("B", "S", "NK", "D")),
    _f("v_cache", IOKind.INOUT, ACT, ("B", "S", "NK", "D")),
    _f("output", IOKind.OUTPUT, ACT, ("B", "NH", "T", "D")),
]

# src/models/optimized_qwen3/shaders/sdpa_decode_cache_write_f32.py:22-170: q and new_k already normalised and
# rotated; new_k / new_v are written at cache_position, then softmax(q K^T / sqrt(D)) V over positions 0..it
SDPA_DECODE_CACHE_WRITE_F32 = _variant("sdpa_decode_cache_write_f32", "SdpaDecodeCacheWriteF32Program",
                                       _SDPA_FIELDS, _sdpa_decode(False, 0.0, kernels.RMS_EPS),
                                       (PushConstantInput("cache_position"),))


def make_sdpa_decode_qk_norm_rope_variant(theta: float, eps: float = kernels.RMS_EPS) -> ShaderVariant:
    """RMS_NORM_ROPE_TRANSPOSE_F16 on q and on k followed by SDPA_DECODE_CACHE_WRITE_F32
    (src/models/optimized_qwen3/dispatch/decode_layer.py:84-109) as one launch: raw q / new_k, their per-head
    RMSNorm weights, RoPE at cache_position with base ``theta``."""
    fields = _SDPA_FIELDS[:3] + [_f("q_norm_weight", IOKind.INPUT, F32, ("D",)),
                                 _f("k_norm_weight", IOKind.INPUT, F32, ("D",))] + _SDPA_FIELDS[3:]
    return _variant("sdpa_decode_qk_norm_rope_cache_write_f32", "SdpaDecodeQkNormRopeCacheWriteProgram", fields,
                    _sdpa_decode(True, theta, eps), (PushConstantInput("cache_position"),))


# Qwen3's RoPE base (config rope_theta 1e6)
SDPA_DECODE_QK_NORM_ROPE_CACHE_WRITE_F32 = make_sdpa_decode_qk_norm_rope_variant(1.0e6)


# ---------------------------------------------------------------- RoPE table, q/k norm + RoPE --

U32 = ("uint32", "int32")  # the reference's uint32 buffers; int32 ones of the same bits are taken too


def _rope_table_launch(rt: RuntimeSession, t, sym, push) -> None:
    kernels.rope_table(t["cos"], t["sin"], push["start_position"], theta=push["theta"])


# src/torch2vk/runtime/rope_table.py:32-122: cos / sin of positions start_position + t.  fp32 tables (the
# reference's are fp16): with them the unfused decode and prefill give the fused kernels' q and k bits.
ROPE_TABLE_F32 = _variant(
    "rope_table_f32", "RopeTableF32Program",
    [_f("cos", IOKind.OUTPUT, F32, ("B", "T", "D")), _f("sin", IOKind.OUTPUT, F32, ("B", "T", "D"))],
    _rope_table_launch, (PushConstantInput("theta", "float32"), PushConstantInput("start_position")))


def _norm_rope_launch(transpose: bool):
    def launch(rt: RuntimeSession, t, sym, push) -> None:
        kernels.rms_norm_rope(t["x"], t["weight"], t["cos"], t["sin"], t["output"], transpose_out=transpose)
    return launch


def _norm_rope(name: str, class_name: str, x_dtype, transpose: bool) -> ShaderVariant:
    out_shape = ("B", "G", "T", "D") if transpose else ("B", "T", "G", "D")
    return _variant(name, class_name, [
        _f("x", IOKind.INPUT, x_dtype, ("B", "T", "G", "D")), _f("weight", IOKind.INPUT, F32, ("D",)),
        _f("cos", IOKind.INPUT, F32, ("B", "T", "D")), _f("sin", IOKind.INPUT, F32, ("B", "T", "D")),
        _f("output", IOKind.OUTPUT, OUT, out_shape)], _norm_rope_launch(transpose))


# src/models/optimized_qwen3/shaders/rms_norm_rope_transpose_f16.py:22-145 (decode q and k, [B, G, T, D] out)
RMS_NORM_ROPE_TRANSPOSE_F16 = _norm_rope("rms_norm_rope_transpose_f16",
                                         "OptimizedQwen3RmsNormRopeTransposeF16Program", OUT, True)
# src/models/optimized_qwen3/shaders/rms_norm_rope_token_f32.py:22-99 (prefill q, token-major out)
RMS_NORM_ROPE_TOKEN_F32 = _norm_rope("rms_norm_rope_token_f32", "OptimizedQwen3RmsNormRopeTokenF32Program", F32,
                                     False)
# src/models/optimized_qwen3/shaders/rms_norm_rope_token_f32_to_f16.py (prefill k, into the cache write)
RMS_NORM_ROPE_TOKEN_F32_TO_F16 = _norm_rope("rms_norm_rope_token_f32_to_f16",
                                            "OptimizedQwen3RmsNormRopeTokenF32ToF16Program", F32, False)


# ------------------------------------------------------------------ LM head + greedy select --

def _lm_head(name: str, class_name: str, layout: str) -> ShaderVariant:
    fields = [_f("x", IOKind.INPUT, ACT, (1, 1, "K")), _weight("weight", "N", layout),
              _f("partial_scores", IOKind.OUTPUT, F32, ("G",)), _f("partial_tokens", IOKind.OUTPUT, U32, ("G",))]

    def launch(rt: RuntimeSession, t, sym, push) -> None:
        kernels.lm_head_argmax_partial(t["x"].view(-1), _bytes(t["weight"]), _LAYOUT_WTYPE[layout],
                                       t["partial_scores"], t["partial_tokens"])

    return _variant(name, class_name, fields, launch)


# src/torch2vk/export/shaders/lm_head_q6_k_argmax_partial_f16.py:24-209: per partial slot the best (score, row)
# of the rows it covers, ties to the lower row; logits are never written.  G is any slot count.
LM_HEAD_Q6_K_ARGMAX_PARTIAL_F16 = _lm_head("lm_head_q6_k_argmax_partial_f16", "LmHeadQ6KArgmaxPartialF16Program",
                                           Q6_K_HALFWORDS)
# The same over a Q4_K head (the uniform-int4 configurations; the reference's Q4_K_M policy always makes the
# head Q6_K, so it has no Q4_K counterpart).
LM_HEAD_Q4_K_ARGMAX_PARTIAL_F16 = _lm_head("lm_head_q4_k_argmax_partial_f16", "LmHeadQ4KArgmaxPartialF16Program",
                                           Q4_K_WORDS)


def _select_chunks_launch(rt: RuntimeSession, t, sym, push) -> None:
    kernels.token_select_chunks(t["scores"], t["tokens"], t["chunk_scores"], t["chunk_tokens"])


# src/torch2vk/export/shaders/qwen3_token_select_reduce_f32.py:22-120: the best pair of each 1024 partials
QWEN3_TOKEN_SELECT_REDUCE_CHUNKS_F32 = _variant(
    "qwen3_token_select_reduce_chunks_f32", "Qwen3TokenSelectReduceChunksF32Program",
    [_f("scores", IOKind.INPUT, F32, ("G",)), _f("tokens", IOKind.INPUT, U32, ("G",)),
     _f("chunk_scores", IOKind.OUTPUT, F32, (ceil_div("G", 1024),)),
     _f("chunk_tokens", IOKind.OUTPUT, U32, (ceil_div("G", 1024),))], _select_chunks_launch)


def _select_launch(rt: RuntimeSession, t, sym, push) -> None:
    kernels.token_select(t["partial_scores"], t["partial_tokens"], t["eos_token_ids"], t["next_token"], t["done"])


# src/torch2vk/export/shaders/qwen3_token_select_reduce_f32.py:123-241: the greedy token (ties to the lowest id)
# and done = it is one of the EOS ids
QWEN3_TOKEN_SELECT_REDUCE_F32 = _variant(
    "qwen3_token_select_reduce_f32", "Qwen3TokenSelectReduceF32Program",
    [_f("partial_scores", IOKind.INPUT, F32, ("G",)), _f("partial_tokens", IOKind.INPUT, U32, ("G",)),
     _f("eos_token_ids", IOKind.INPUT, "int64", ("E",)), _f("next_token", IOKind.OUTPUT, "int64", (1, 1)),
     _f("done", IOKind.OUTPUT, U32, (1,))], _select_launch)


def _token_store_launch(stop_on_eos: bool):
    def launch(rt: RuntimeSession, t, sym, push) -> None:
        idx = push["token_index"]
        kernels.token_store(t["next_token"], t["done"], t["generated_tokens"].view(-1), t["generated_length"],
                            t["stopped"], stop_on_eos=stop_on_eos,
                            token_index=0 if isinstance(idx, torch.Tensor) else int(idx),
                            token_index_ptr=idx if isinstance(idx, torch.Tensor) else None)
    return launch


def make_qwen3_token_store_variant(name: str, class_name: str, stop_on_eos: bool) -> ShaderVariant:
    """generated_tokens[token_index] = next_token and generated_length = token_index + 1 unless stopped; with
    ``stop_on_eos`` a selected EOS (done) also sets stopped (src/torch2vk/export/shaders/qwen3_token_store.py)."""
    return _variant(name, class_name, [
        _f("next_token", IOKind.INPUT, "int64", (1, 1)), _f("done", IOKind.INPUT, U32, (1,)),
        _f("generated_tokens", IOKind.INOUT, "int64", (1, "G")), _f("generated_length", IOKind.INOUT, U32, (1,)),
        _f("stopped", IOKind.INOUT, U32, (1,))], _token_store_launch(stop_on_eos), (PushConstantInput("token_index"),))


# src/torch2vk/export/shaders/qwen3_token_store.py:19 and :124; src/models/optimized_qwen3/shaders/
# qwen3_token_store_eos_f32.py (stop_on_eos pushed as 1)
QWEN3_TOKEN_STORE = make_qwen3_token_store_variant("qwen3_token_store", "Qwen3TokenStoreProgram", False)
QWEN3_TOKEN_STORE_EOS = make_qwen3_token_store_variant("qwen3_token_store_eos", "Qwen3TokenStoreEosProgram", True)
QWEN3_TOKEN_STORE_EOS_F32 = make_qwen3_token_store_variant("qwen3_token_store_eos_f32",
                                                           "Qwen3TokenStoreEosF32Program", True)


def _embed_q8_launch(rt: RuntimeSession, t, sym, push) -> None:
    kernels.embedding_q8_0(_bytes(t["weight"]), t["indices"].view(-1), sym["H"], out=t["output"].view(-1, sym["H"]))


# src/models/quantized_qwen3_asr/shaders/embedding_q8_0_f32.py:25-97 (the Qwen3-ASR policy's token embedding)
EMBEDDING_Q8_0_F32 = _variant(
    "embedding_q8_0_f32", "EmbeddingQ8_0Program",
    [_weight("weight", "V", Q8_0_HALFWORDS, "H"), _f("indices", IOKind.INPUT, "int64", ("B", "T")),
     _f("output", IOKind.OUTPUT, F32, ("B", "T", "H"))], _embed_q8_launch)

# src/models/optimized_qwen3/shaders/embedding_q4_k_act_f32.py:21-60 (the prefill chunks' embedding)
EMBEDDING_Q4_K_ACT_F32 = _variant(
    "embedding_q4_k_act_f32", "OptimizedQwen3EmbeddingQ4KActF32Program",
    [_weight("weight", "V", Q4_K_WORDS, "H"), _f("indices", IOKind.INPUT, "int64", ("I0", "I1")),
     _f("output", IOKind.OUTPUT, F32, ("I0", "I1", "H"))],
    lambda rt, t, sym, push: kernels.embedding_q4_k(_bytes(t["weight"]), t["indices"].view(-1), sym["H"],
                                                    out=t["output"].view(-1, sym["H"])))


# ------------------------------------------------------------------------- prefill operators --

# src/models/optimized_qwen3/shaders/rms_norm_mul_f32.py:22-40 (fp32 rows in; bf16 out for the GEMMs)
RMS_NORM_MUL_F32 = _variant(
    "rms_norm_mul_f32", "OptimizedQwen3RmsNormMulF32Program",
    [_f("x", IOKind.INPUT, F32, ("B", "T", "H")), _f("weight", IOKind.INPUT, F32, ("H",)),
     _f("output", IOKind.OUTPUT, OUT, ("B", "T", "H"))], _rms_launch)


def _llama_matmul(name: str, class_name: str, layout: str) -> ShaderVariant:
    """The prefill GEMM of a K-quant weight (src/models/optimized_qwen3/shaders/llama_matmul_q4_k_f32.py:32-141):
    the _M and _L names are the reference's tile sizes for <= 320 and more tokens; here both run the matrix-core
    GEMM, which picks its own tiles (and splits K for small grids)."""
    fields = [_weight("weight", "N", layout), _f("x", IOKind.INPUT, ACT, ("X0", "X1", "K")),
              _f("output", IOKind.OUTPUT, OUT, ("X0", "X1", "N"))]

    def launch(rt: RuntimeSession, t, sym, push) -> None:
        kernels.gemm(t["x"], _bytes(t["weight"]), _LAYOUT_WTYPE[layout], out=t["output"])

    return _variant(name, class_name, fields, launch)


LLAMA_MATMUL_Q4_K_F32_M = _llama_matmul("llama_matmul_q4_k_f32_m", "LlamaMatmulQ4KF32Program", Q4_K_WORDS)
LLAMA_MATMUL_Q4_K_F32_L = _llama_matmul("llama_matmul_q4_k_f32_l", "LlamaMatmulQ4KF32Program", Q4_K_WORDS)
LLAMA_MATMUL_Q6_K_F32_M = _llama_matmul("llama_matmul_q6_k_f32_m", "LlamaMatmulQ6KF32Program", Q6_K_HALFWORDS)
LLAMA_MATMUL_Q6_K_F32_L = _llama_matmul("llama_matmul_q6_k_f32_l", "LlamaMatmulQ6KF32Program", Q6_K_HALFWORDS)


def _add_launch(rt: RuntimeSession, t, sym, push) -> None:
    kernels.add(t["x"], t["y"], out=t["output"])


# src/models/optimized_qwen3/shaders/add_f32_prefill.py:20-60 (the prefill residual adds)
ADD_F32_PREFILL = _variant(
    "add_f32_prefill", "AddF32PrefillProgram",
    [_f("x", IOKind.INPUT, F32, (1, "T", "H")), _f("y", IOKind.INPUT, F32, (1, "T", "H")),
     _f("output", IOKind.OUTPUT, F32, (1, "T", "H"))], _add_launch)
# src/models/optimized_qwen3/shaders/add_f32_36.py:22-80 (the last prefill layer's residual add on the last token;
# the reference adds in fp16, here fp32 or bf16)
ADD_F32_36 = _variant(
    "add_f32_36", "ExportAddF32Program",
    [_f("x", IOKind.INPUT, OUT, (1, "T", "H")), _f("y", IOKind.INPUT, OUT, (1, "T", "H")),
     _f("output", IOKind.OUTPUT, OUT, (1, "T", "H"))], _add_launch)

# src/models/optimized_qwen3/shaders/slice_last_token_f32_to_f16.py:19-60 (fp32 or bf16 out; the decoder keeps the
# residual stream in fp32)
SLICE_LAST_TOKEN_F32_TO_F16 = _variant(
    "slice_last_token_f32_to_f16", "SliceLastTokenF32ToF16Program",
    [_f("x", IOKind.INPUT, F32, ("B", "S", "H")), _f("output", IOKind.OUTPUT, OUT, ("B", 1, "H"))],
    lambda rt, t, sym, push: kernels.slice_last_token(t["x"], t["output"]))

# src/models/optimized_qwen3/shaders/swiglu_f32.py:20-60 (fp32 gate / up; bf16 out, the down GEMM's input)
SWIGLU_F32 = _variant(
    "swiglu_f32", "SwigluF32Program",
    [_f("gate", IOKind.INPUT, F32, ("B", "T", "H")), _f("up", IOKind.INPUT, F32, ("B", "T", "H")),
     _f("output", IOKind.OUTPUT, ACT, ("B", "T", "H"))], _swiglu_launch)


def _kv_write(name: str, class_name: str, src_dtype, n_caches: int) -> ShaderVariant:
    names = ("cache_a", "cache_b", "cache_c")[:n_caches]
    fields = [_f(n, IOKind.INOUT, ACT, ("B", f"S{n[-1].upper()}", "H", "D")) for n in names]
    fields += [_f("cache_position", IOKind.INPUT, "int64", ("T",)),
               _f("src", IOKind.INPUT, src_dtype, ("B", "T", "H", "D"))]

    def launch(rt: RuntimeSession, t, sym, push) -> None:
        kernels.kv_cache_write(t["src"], t["cache_position"], [t[n] for n in names])

    return _variant(name, class_name, fields, launch)


# src/models/optimized_qwen3/shaders/token_major_kv_cache_write_f16_pair.py:20-103 and the _triple / value forms:
# rows src[b, t] to cache row cache_position[t] of every cache (bf16 caches; the reference's are fp16)
TOKEN_MAJOR_KV_CACHE_WRITE_F16_PAIR = _kv_write("token_major_kv_cache_write_f16_pair",
                                                "OptimizedQwen3TokenMajorKvCacheWriteF16PairProgram", ACT, 2)
TOKEN_MAJOR_KV_CACHE_WRITE_F16_TRIPLE = _kv_write("token_major_kv_cache_write_f16_triple",
                                                  "OptimizedQwen3TokenMajorKvCacheWriteF16TripleProgram", ACT, 3)
TOKEN_MAJOR_VALUE_CACHE_WRITE_F32_TO_F16_PAIR = _kv_write(
    "token_major_value_cache_write_f32_to_f16_pair", "OptimizedQwen3TokenMajorValueCacheWriteF32ToF16PairProgram",
    F32, 2)
TOKEN_MAJOR_VALUE_CACHE_WRITE_F32_TO_F16_TRIPLE = _kv_write(
    "token_major_value_cache_write_f32_to_f16_triple",
    "OptimizedQwen3TokenMajorValueCacheWriteF32ToF16TripleProgram", F32, 3)

# tile classes of a [T, S] additive mask: uint8 [1, ceil(T / 128), ceil(S / 64)] (the reference packs them into
# uint32 [W, R]); 1 all masked, 2 all zero, 0 mixed
_MASK_OPT = ("uint8", (1, ceil_div("T", kernels.FA_BLOCK_QUERIES), ceil_div("S", kernels.FA_TILE_KEYS)))


def _mask_opt_launch(rt: RuntimeSession, t, sym, push) -> None:
    kernels.fa_mask_tiles(t["mask"].unsqueeze(0), out=t["output"])


# src/models/optimized_qwen3/shaders/fa_mask_opt_f16.py:22-60 (fp32 additive mask here; the reference's is fp16)
FA_MASK_OPT_F16 = _variant(
    "fa_mask_opt_f16", "OptimizedQwen3FaMaskOptF16Program",
    [_f("mask", IOKind.INPUT, F32, ("T", "S")), _f("output", IOKind.OUTPUT, *_MASK_OPT)], _mask_opt_launch)


def _flash_launch(rt: RuntimeSession, t, sym, push) -> None:
    kernels.flash_attn_prefill(t["q"], t["k"], t["v"], out=t["output"], causal=False, mask=t["mask"].unsqueeze(0),
                               mask_tiles=t["mask_opt"])


# src/models/optimized_qwen3/shaders/llama_flash_attn_f32_f16_f16.py:35-175: softmax(q k^T / sqrt(D) + mask) v
# over token-major q [B, T, NH, D] and caches [B, S, NK, D], GQA; mask_opt's all-masked tiles are skipped and
# all-zero ones not read.  The reference binds q as its "sink" but its mask_n_head_log2 push (NH) leaves sinks off,
# so the field is checked and not read.
LLAMA_FLASH_ATTN_F32_F16_F16 = _variant(
    "llama_flash_attn_f32_f16_f16", "LlamaFlashAttnF32F16F16Program",
    [_f("q", IOKind.INPUT, ACT, ("B", "T", "NH", "D")), _f("k", IOKind.INPUT, ACT, ("B", "S", "NK", "D")),
     _f("v", IOKind.INPUT, ACT, ("B", "S", "NK", "D")), _f("mask", IOKind.INPUT, F32, ("T", "S")),
     _f("sink", IOKind.INPUT, OUT, ("B", "T", "NH", "D")), _f("output", IOKind.OUTPUT, ACT, ("B", "T", "NH", "D")),
     _f("mask_opt", IOKind.INPUT, *_MASK_OPT)], _flash_launch)
