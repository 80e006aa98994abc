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
