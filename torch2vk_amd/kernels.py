"""Checked torch-tensor wrappers over the libt2h C ABI.

Each function validates device, dtype, shape, contiguity and alignment on the
host (the reference does the same before a launch, src/torch2vk/runtime/dispatcher.py:35-53)
and then enqueues one C-ABI call on the current HIP stream.  Nothing here
computes on the CPU: there is no fallback path.
"""

from __future__ import annotations

import ctypes

import torch

from torch2vk_amd import _lib
from torch2vk_amd._lib import T2H_DTYPE_BF16, T2H_DTYPE_F32, call, ptr, stream_handle

Q4_K_BYTES = 144
Q6_K_BYTES = 210
Q8_0_BYTES = 34
RMS_EPS = 1e-6

_OUT_DTYPES = {torch.float32: T2H_DTYPE_F32, torch.bfloat16: T2H_DTYPE_BF16}
# the reference's uint32 buffers (token ids of the LM head's partials, done / length / stopped flags), or
# int32 ones of the same bits
_TOKEN_DTYPES = (torch.int32, torch.uint32)
WTYPES = {"q4_k": _lib.T2H_WTYPE_Q4_K, "q6_k": _lib.T2H_WTYPE_Q6_K, "q8_0": _lib.T2H_WTYPE_Q8_0,
          "bf16": _lib.T2H_WTYPE_BF16}


def _check(t: torch.Tensor, name: str, dtype: torch.dtype | tuple[torch.dtype, ...], *, align: int = 16) -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor, got {type(t).__name__}")
    if t.device.type != "cuda":
        raise ValueError(f"{name} must live on a HIP device, got {t.device}")
    dtypes = dtype if isinstance(dtype, tuple) else (dtype,)
    if t.dtype not in dtypes:
        raise TypeError(f"{name} dtype {t.dtype} not in {dtypes}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if t.data_ptr() % align:
        raise ValueError(f"{name} must be {align}-byte aligned")


def q4_k_row_bytes(k: int) -> int:
    if k % 256:
        raise ValueError(f"Q4_K needs K % 256 == 0, got {k}")
    return k // 256 * Q4_K_BYTES


def _check_q4(w: torch.Tensor, name: str, n: int | None, k: int) -> int:
    _check(w, name, torch.uint8)
    if w.dim() != 2 or w.shape[1] != q4_k_row_bytes(k):
        raise ValueError(f"{name} must be uint8 [N, {q4_k_row_bytes(k)}] for K={k}, got {tuple(w.shape)}")
    if n is not None and w.shape[0] != n:
        raise ValueError(f"{name} has {w.shape[0]} rows, expected {n}")
    return int(w.shape[0])


# ------------------------------------------------------------ quantizers --


def quantize(x: torch.Tensor, wtype: str) -> torch.Tensor:
    """fp32 [R, K] -> packed GGUF rows (uint8), bit-identical to the CPU oracle."""
    _check(x, "x", torch.float32)
    if x.dim() != 2:
        raise ValueError(f"x must be rank 2, got {tuple(x.shape)}")
    rows, k = x.shape
    if wtype == "q8_0":
        padded = (k + 31) // 32 * 32
        if padded != k:
            x = torch.nn.functional.pad(x, (0, padded - k)).contiguous()
        out = torch.empty(rows, padded // 32 * Q8_0_BYTES, dtype=torch.uint8, device=x.device)
        call("t2h_quantize_q8_0", ptr(x), rows, padded, ptr(out), stream_handle())
        return out
    if k % 256:
        raise ValueError(f"{wtype} needs K % 256 == 0, got {k}")
    if wtype == "q4_k":
        out = torch.empty(rows, k // 256 * Q4_K_BYTES, dtype=torch.uint8, device=x.device)
        call("t2h_quantize_q4_k", ptr(x), rows, k, ptr(out), stream_handle())
    elif wtype == "q6_k":
        out = torch.empty(rows, k // 256 * Q6_K_BYTES, dtype=torch.uint8, device=x.device)
        call("t2h_quantize_q6_k", ptr(x), rows, k, ptr(out), stream_handle())
    else:
        raise ValueError(f"unknown weight type {wtype!r}")
    return out


def dequantize(w: torch.Tensor, wtype: str, k: int) -> torch.Tensor:
    """Packed GGUF rows -> fp32 [R, K]."""
    _check(w, "w", torch.uint8, align=1)
    rows = int(w.shape[0])
    out = torch.empty(rows, k, dtype=torch.float32, device=w.device)
    call("t2h_dequantize", WTYPES[wtype], ptr(w), rows, k, ptr(out), stream_handle())
    return out


# ------------------------------------------------------------ GEMV family --


def q4k_matvec(x: torch.Tensor, w: torch.Tensor, *, out: torch.Tensor | None = None,
               out_dtype: torch.dtype = torch.float32, residual: torch.Tensor | None = None) -> torch.Tensor:
    """y[M, N] = x[M, K] . deq(W)^T (+ residual); x bf16."""
    _check(x, "x", torch.bfloat16)
    k = int(x.shape[-1])
    m = x.numel() // k
    n = _check_q4(w, "weight", None, k)
    if out is None:
        out = torch.empty(*x.shape[:-1], n, dtype=out_dtype, device=x.device)
    _check(out, "output", tuple(_OUT_DTYPES), align=4)
    if out.numel() != m * n:
        raise ValueError(f"output has {out.numel()} elements, expected {m * n}")
    if residual is not None:
        _check(residual, "residual", torch.float32, align=4)
        if residual.numel() != m * n or out.dtype != torch.float32:
            raise ValueError("residual must be fp32 with the output's shape; output must be fp32")
    call("t2h_q4k_matvec", ptr(x), ptr(w), ptr(out), _OUT_DTYPES[out.dtype], ptr(residual), m, k, n,
         stream_handle())
    return out


def _ptr_array(values):
    arr = (_lib.ctypes.c_void_p * len(values))(*values)
    return arr


def q4k_matvec_multi(x: torch.Tensor, weights: list[torch.Tensor], outs: list[torch.Tensor], *,
                     norm_weight: torch.Tensor | None = None, eps: float = RMS_EPS) -> None:
    """Q|K|V (or gate|up) sharing one x; with norm_weight, x is the fp32 residual stream normalised in-kernel."""
    if norm_weight is None:
        _check(x, "x", torch.bfloat16)
    else:
        _check(x, "x", torch.float32)
        _check(norm_weight, "norm_weight", torch.float32)
        if norm_weight.numel() != x.numel():
            raise ValueError("norm_weight must have K elements")
    k = int(x.numel())
    if len(weights) != len(outs) or not 1 <= len(weights) <= 3:
        raise ValueError("need 1..3 weights and as many outputs")
    ns = []
    out_dtype = outs[0].dtype
    for i, (w, o) in enumerate(zip(weights, outs)):
        n = _check_q4(w, f"weight[{i}]", None, k)
        _check(o, f"output[{i}]", out_dtype, align=4)
        if o.numel() != n:
            raise ValueError(f"output[{i}] has {o.numel()} elements, expected {n}")
        ns.append(n)
    if out_dtype not in _OUT_DTYPES:
        raise TypeError(f"unsupported output dtype {out_dtype}")
    wp = _ptr_array([ptr(w) for w in weights])
    yp = _ptr_array([ptr(o) for o in outs])
    nn = (_lib.ctypes.c_uint32 * len(ns))(*ns)
    call("t2h_q4k_matvec_multi", ptr(x), ptr(norm_weight), eps, len(weights), wp, yp, nn, k,
         _OUT_DTYPES[out_dtype], stream_handle())


def q4k_rmsnorm_swiglu(h: torch.Tensor, norm_weight: torch.Tensor, w_gate: torch.Tensor, w_up: torch.Tensor,
                       out: torch.Tensor, eps: float = RMS_EPS) -> torch.Tensor:
    """act = silu(g) * u, g|u = RMSNorm(h) . deq(W_gate|W_up)^T; act bf16 [N]."""
    _check(h, "h", torch.float32)
    _check(norm_weight, "norm_weight", torch.float32)
    k = int(h.numel())
    n = _check_q4(w_gate, "gate_weight", None, k)
    _check_q4(w_up, "up_weight", n, k)
    _check(out, "output", torch.bfloat16, align=4)
    if out.numel() != n:
        raise ValueError(f"output must have {n} elements")
    call("t2h_q4k_rmsnorm_swiglu_matvec", ptr(h), ptr(norm_weight), eps, ptr(w_gate), ptr(w_up), ptr(out), k, n,
         stream_handle())
    return out


def q4k_lm_head_argmax_partial(x: torch.Tensor, w: torch.Tensor, partial_scores: torch.Tensor,
                               partial_tokens: torch.Tensor, *, norm_weight: torch.Tensor | None = None,
                               eps: float = RMS_EPS) -> None:
    if norm_weight is None:
        _check(x, "x", torch.bfloat16)
    else:
        _check(x, "x", torch.float32)
        _check(norm_weight, "norm_weight", torch.float32)
    k = int(x.numel())
    n = _check_q4(w, "weight", None, k)
    _check(partial_scores, "partial_scores", torch.float32, align=4)
    _check(partial_tokens, "partial_tokens", _TOKEN_DTYPES, align=4)
    g = int(partial_scores.numel())
    if partial_tokens.numel() != g or g == 0:
        raise ValueError("partial_scores and partial_tokens must have the same non-zero length")
    call("t2h_q4k_lm_head_argmax_partial", ptr(x), ptr(norm_weight), eps, ptr(w), k, n, ptr(partial_scores),
         ptr(partial_tokens), g, stream_handle())


def q4k_lm_head_argmax_partial_seqs(hs: list[torch.Tensor], w: torch.Tensor, partial_scores: list[torch.Tensor],
                                    partial_tokens: list[torch.Tensor], *, norm_weight: torch.Tensor,
                                    eps: float = RMS_EPS) -> None:
    """q4k_lm_head_argmax_partial (final RMSNorm fused) for 1..4 sequences in one launch: the head is read
    once; sequence i's partials land in partial_scores[i] / partial_tokens[i], bit-identical to its own
    call (t2h_q4k_lm_head_argmax_partial_seqs)."""
    n_seq = len(hs)
    if not 1 <= n_seq <= LM_HEAD_SEQS_MAX or len(partial_scores) != n_seq or len(partial_tokens) != n_seq:
        raise ValueError(f"1..{LM_HEAD_SEQS_MAX} sequences with one partial pair each")
    _check(norm_weight, "norm_weight", torch.float32)
    k = int(hs[0].numel())
    for h in hs:
        _check(h, "h", torch.float32)
        if h.numel() != k:
            raise ValueError("every h must have the same length")
    n = _check_q4(w, "weight", None, k)
    g = int(partial_scores[0].numel())
    for sc, tk in zip(partial_scores, partial_tokens):
        _check(sc, "partial_scores", torch.float32, align=4)
        _check(tk, "partial_tokens", _TOKEN_DTYPES, align=4)
        if sc.numel() != g or tk.numel() != g or g == 0:
            raise ValueError("partial_scores and partial_tokens must all have the same non-zero length")
    arr = lambda ts: (ctypes.c_void_p * n_seq)(*[t.data_ptr() for t in ts])  # noqa: E731
    h_arr, s_arr, t_arr = arr(hs), arr(partial_scores), arr(partial_tokens)
    call("t2h_q4k_lm_head_argmax_partial_seqs", n_seq, ctypes.addressof(h_arr), ptr(norm_weight), eps, ptr(w), k,
         n, ctypes.addressof(s_arr), ctypes.addressof(t_arr), g, stream_handle())


_BLOCK = {"q4_k": (256, Q4_K_BYTES), "q6_k": (256, Q6_K_BYTES), "q8_0": (32, Q8_0_BYTES)}


def row_bytes(wtype: str, k: int) -> int:
    values, nbytes = _BLOCK[wtype]
    if k % values:
        raise ValueError(f"{wtype} needs K % {values} == 0, got {k}")
    return k // values * nbytes


def _check_packed(w: torch.Tensor, name: str, wtype: str, k: int) -> int:
    if wtype == "bf16":
        _check(w, name, torch.bfloat16)
        if w.dim() != 2 or w.shape[1] != k:
            raise ValueError(f"{name} must be bf16 [N, {k}], got {tuple(w.shape)}")
        return int(w.shape[0])
    _check(w, name, torch.uint8)
    rb = row_bytes(wtype, k)
    if w.dim() != 2 or w.shape[1] != rb:
        raise ValueError(f"{name} must be uint8 [N, {rb}] ({wtype}, K={k}), got {tuple(w.shape)}")
    return int(w.shape[0])


def qx_matvec(x: torch.Tensor, w: torch.Tensor, wtype: str, *, out: torch.Tensor | None = None,
              out_dtype: torch.dtype = torch.float32, residual: torch.Tensor | None = None,
              norm_weight: torch.Tensor | None = None, eps: float = RMS_EPS) -> torch.Tensor:
    """Q6_K / Q8_0 GEMV: y[M, N] = x[M, K] . deq(W)^T (+ residual).  x bf16, or (Q6_K with
    norm_weight) the fp32 residual stream [K] normalised in-kernel."""
    if wtype not in ("q6_k", "q8_0"):
        raise ValueError(f"qx_matvec handles q6_k and q8_0, got {wtype!r}")
    if norm_weight is None:
        _check(x, "x", torch.bfloat16)
    else:
        if wtype != "q6_k" or residual is not None:
            raise ValueError("the fused RMSNorm prologue is built for Q6_K without residual")
        _check(x, "x", torch.float32)
        _check(norm_weight, "norm_weight", torch.float32)
        if norm_weight.numel() != x.numel():
            raise ValueError("norm_weight must have K elements")
    k = int(x.shape[-1])
    m = x.numel() // k
    if norm_weight is not None and m != 1:
        raise ValueError("the fused RMSNorm prologue takes one token")
    n = _check_packed(w, "weight", wtype, k)
    if out is None:
        out = torch.empty(*x.shape[:-1], n, dtype=out_dtype, device=x.device)
    _check(out, "output", tuple(_OUT_DTYPES), align=4)
    if out.numel() != m * n:
        raise ValueError(f"output has {out.numel()} elements, expected {m * n}")
    if residual is not None:
        _check(residual, "residual", torch.float32, align=4)
        if residual.numel() != m * n or out.dtype != torch.float32:
            raise ValueError("residual must be fp32 with the output's shape; output must be fp32")
    if norm_weight is not None:
        call("t2h_q6k_rmsnorm_matvec", ptr(x), ptr(norm_weight), eps, ptr(w), ptr(out), _OUT_DTYPES[out.dtype],
             k, n, stream_handle())
    else:
        name = "t2h_q6k_matvec" if wtype == "q6_k" else "t2h_q8_0_matvec"
        call(name, ptr(x), ptr(w), ptr(out), _OUT_DTYPES[out.dtype], ptr(residual), m, k, n, stream_handle())
    return out


def lm_head_argmax_partial(x: torch.Tensor, w: torch.Tensor, wtype: str, partial_scores: torch.Tensor,
                           partial_tokens: torch.Tensor, *, norm_weight: torch.Tensor | None = None,
                           eps: float = RMS_EPS) -> None:
    """LM head GEMV + per-block argmax for a Q4_K or Q6_K head (logits never materialised)."""
    if wtype == "q4_k":
        q4k_lm_head_argmax_partial(x, w, partial_scores, partial_tokens, norm_weight=norm_weight, eps=eps)
        return
    if wtype != "q6_k":
        raise ValueError(f"LM head argmax is built for q4_k and q6_k, got {wtype!r}")
    if norm_weight is None:
        _check(x, "x", torch.bfloat16)
    else:
        _check(x, "x", torch.float32)
        _check(norm_weight, "norm_weight", torch.float32)
    k = int(x.numel())
    n = _check_packed(w, "weight", "q6_k", k)
    _check(partial_scores, "partial_scores", torch.float32, align=4)
    _check(partial_tokens, "partial_tokens", _TOKEN_DTYPES, align=4)
    g = int(partial_scores.numel())
    if partial_tokens.numel() != g or g == 0:
        raise ValueError("partial_scores and partial_tokens must have the same non-zero length")
    call("t2h_q6k_lm_head_argmax_partial", ptr(x), ptr(norm_weight), eps, ptr(w), k, n, ptr(partial_scores),
         ptr(partial_tokens), g, stream_handle())


GEMM_FILL_BLOCKS = 128  # grids below this many tiles split K (t2h_gemm_splitk)
# From this many rows of x, a one-pass prefill GEMM dequantises its packed weights once into a bf16 scratch
# (t2h_dequantize_bf16, ~1 ns per weight) and runs the tile loop on bf16 rows, instead of dequantising every
# weight tile once per 256 rows of x inside the loop (measured on MI355X at M 16384, K 4096, N 12288 Q8_0: 1.85 ms
# in-loop against 0.05 + 1.52 ms; break-even near 2300 rows).  The products are bit-identical either way.
# 0 disables it.
DEQUANT_FIRST_ROWS = 4096


def _dequant_first(m: int, wtype: str, splits: int) -> bool:
    return DEQUANT_FIRST_ROWS > 0 and m >= DEQUANT_FIRST_ROWS and splits == 1 and wtype != "bf16"


def gemm_splits(m: int, n_cols: int, k: int) -> int:
    """K parts for a prefill GEMM of m rows and n_cols tile columns (1 = the one-pass GEMM): when the
    one-pass grid has fewer than GEMM_FILL_BLOCKS tiles, enough parts that the split grid (128-row tiles)
    reaches ~256 blocks, each part at least 2 stages of 64, at most 16 parts."""
    tiles_n = -(-n_cols // 256)
    tiles_256 = -(-m // 256) * tiles_n
    tiles = -(-m // 128) * tiles_n if (tiles_256 < 1024 and m > 128) else tiles_256
    if tiles >= GEMM_FILL_BLOCKS:
        return 1
    split_tiles = -(-m // 128) * tiles_n
    return max(1, min(k // 128, -(-256 // split_tiles), 16))


def _gemm_splitk(wtype: str, x: torch.Tensor, w: torch.Tensor, w_up: torch.Tensor | None, out: torch.Tensor,
                 m: int, k: int, n: int, w_k: int, splits: int, *, bias: torch.Tensor | None = None, act: int = 0,
                 residual: torch.Tensor | None = None) -> None:
    nbytes = int(_lib.lib().t2h_gemm_splitk_bytes(m, n, splits, 1 if w_up is not None else 0))
    partials = torch.empty(nbytes // 4, dtype=torch.float32, device=x.device)
    call("t2h_gemm_splitk", WTYPES[wtype], ptr(x), ptr(w), ptr(w_up), ptr(bias), act, ptr(out),
         _OUT_DTYPES[out.dtype], ptr(residual), m, k, n, w_k, splits, ptr(partials), nbytes, stream_handle())


def gemm(x: torch.Tensor, w: torch.Tensor, wtype: str, *, out: torch.Tensor | None = None,
         out_dtype: torch.dtype = torch.bfloat16, residual: torch.Tensor | None = None,
         splits: int | None = None) -> torch.Tensor:
    """Prefill GEMM on the matrix cores: y[M, N] = x[M, K] . deq(W)^T (+ residual); x bf16, W Q8_0, Q4_K or
    Q6_K packed rows, or bf16 [N, K] ("bf16", e.g. from :func:`dequantize_bf16`).  ``splits``: K parts
    (t2h_gemm_splitk; None = gemm_splits' choice, 1 = one pass)."""
    if wtype not in ("q8_0", "q4_k", "q6_k", "bf16"):
        raise ValueError(f"gemm handles q8_0, q4_k, q6_k and bf16 weights, got {wtype!r}")
    _check(x, "x", torch.bfloat16)
    k = int(x.shape[-1])
    if k % 64:
        raise ValueError(f"gemm needs K % 64 == 0, got {k}")
    m = x.numel() // k
    n = _check_packed(w, "weight", wtype, k)
    if out is None:
        out = torch.empty(*x.shape[:-1], n, dtype=out_dtype, device=x.device)
    _check(out, "output", tuple(_OUT_DTYPES), align=4)
    if out.numel() != m * n:
        raise ValueError(f"output has {out.numel()} elements, expected {m * n}")
    if residual is not None:
        _check(residual, "residual", torch.float32, align=4)
        if residual.numel() != m * n or out.dtype != torch.float32:
            raise ValueError("residual must be fp32 with the output's shape; output must be fp32")
    splits = gemm_splits(m, n, k) if splits is None else splits
    if splits > 1:
        _gemm_splitk(wtype, x, w, None, out, m, k, n, k, splits, residual=residual)
        return out
    if _dequant_first(m, wtype, splits):
        w, wtype = dequantize_bf16(w, wtype, k), "bf16"
    name = {"q8_0": "t2h_q8_0_gemm", "q4_k": "t2h_q4k_gemm", "q6_k": "t2h_q6k_gemm", "bf16": "t2h_bf16_gemm"}[wtype]
    call(name, ptr(x), ptr(w), ptr(out), _OUT_DTYPES[out.dtype], ptr(residual), m, k, n, stream_handle())
    return out


def gemm_swiglu(x: torch.Tensor, w_gate: torch.Tensor, w_up: torch.Tensor, wtype: str, *,
                out: torch.Tensor | None = None, splits: int | None = None) -> torch.Tensor:
    """bf16 [M, F] = silu(x . deq(W_gate)^T) * (x . deq(W_up)^T) in one matrix-core launch (the prefill MLP's
    gate and up GEMMs with SwiGLU in the epilogue); x bf16 [M, K], both weights [F, K] of type ``wtype``.
    ``splits`` as for :func:`gemm` (split-K: the products, then SwiGLU in the reduction)."""
    if wtype not in ("q8_0", "q4_k", "q6_k", "bf16"):
        raise ValueError(f"gemm_swiglu handles q8_0, q4_k, q6_k and bf16 weights, got {wtype!r}")
    _check(x, "x", torch.bfloat16)
    k = int(x.shape[-1])
    if k % 64:
        raise ValueError(f"gemm_swiglu needs K % 64 == 0, got {k}")
    m = x.numel() // k
    n = _check_packed(w_gate, "w_gate", wtype, k)
    if _check_packed(w_up, "w_up", wtype, k) != n:
        raise ValueError("w_gate and w_up must have the same number of rows")
    if out is None:
        out = torch.empty(*x.shape[:-1], n, dtype=torch.bfloat16, device=x.device)
    _check(out, "output", torch.bfloat16, align=2)
    if out.numel() != m * n:
        raise ValueError(f"output has {out.numel()} elements, expected {m * n}")
    splits = gemm_splits(m, 2 * n, k) if splits is None else splits
    if splits > 1:
        _gemm_splitk(wtype, x, w_gate, w_up, out, m, k, n, k, splits)
        return out
    if _dequant_first(m, wtype, splits):
        w_gate, w_up, wtype = dequantize_bf16(w_gate, wtype, k), dequantize_bf16(w_up, wtype, k), "bf16"
    call("t2h_gemm_swiglu", WTYPES[wtype], ptr(x), ptr(w_gate), ptr(w_up), ptr(out), m, k, n, stream_handle())
    return out


def dequantize_bf16(w: torch.Tensor, wtype: str, k: int, *, out: torch.Tensor | None = None) -> torch.Tensor:
    """bf16 [N, K] = the values the prefill GEMMs dequantise W's packed rows to (t2h_dequantize_bf16): a GEMM
    with wtype "bf16" over the result equals the quantized GEMM over W bit for bit."""
    if wtype not in ("q8_0", "q4_k", "q6_k"):
        raise ValueError(f"dequantize_bf16 handles q8_0, q4_k and q6_k weights, got {wtype!r}")
    if k % 64:
        raise ValueError(f"dequantize_bf16 needs K % 64 == 0, got {k}")
    n = _check_packed(w, "weight", wtype, k)
    if out is None:
        out = torch.empty(n, k, dtype=torch.bfloat16, device=w.device)
    _check(out, "output", torch.bfloat16)
    if out.numel() != n * k:
        raise ValueError(f"output has {out.numel()} elements, expected {n * k}")
    call("t2h_dequantize_bf16", WTYPES[wtype], ptr(w), n, k, ptr(out), stream_handle())
    return out


GEMV_MAX_ROWS = 8  # rows handled by the decode GEMVs; more go to the matrix-core GEMM


def matvec_supported(wtype: str, k: int, n: int) -> bool:
    """Whether the decode GEMV of ``wtype`` is built for rows of k values and n output rows."""
    return bool(_lib.lib().t2h_matvec_supported(WTYPES[wtype], k, n))


def quantized_linear(x: torch.Tensor, w: torch.Tensor, wtype: str, *, out: torch.Tensor | None = None,
                     out_dtype: torch.dtype = torch.float32, residual: torch.Tensor | None = None) -> torch.Tensor:
    """y[M, N] = x[M, K] . deq(W)^T (+ residual) with the kernel the reference would pick: the weight's GGUF type
    selects the family (run_quantized_linear, src/torch2vk/runtime/quantized_dispatch.py:15-35) and M <= 8 rows
    run the decode GEMV (one launch per row, the weights streamed per row), more the matrix-core GEMM
    (make_linear_nobias_q4_k_m_variant, src/torch2vk/export/shaders/linear_nobias_quantized.py:47-80).
    Shapes the GEMVs are not built for (matvec_supported) run on the GEMM at any M."""
    if wtype not in ("q4_k", "q6_k", "q8_0"):
        raise ValueError(f"quantized_linear handles q4_k, q6_k and q8_0 weights, got {wtype!r}")
    k = int(x.shape[-1])
    m = x.numel() // k if k else 0
    n = int(w.shape[0])
    if m <= GEMV_MAX_ROWS and matvec_supported(wtype, k, n):
        if wtype == "q4_k":
            return q4k_matvec(x, w, out=out, out_dtype=out_dtype, residual=residual)
        return qx_matvec(x, w, wtype, out=out, out_dtype=out_dtype, residual=residual)
    return gemm(x, w, wtype, out=out, out_dtype=out_dtype, residual=residual)


def qk_norm_rope_cache(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, q_out: torch.Tensor,
                       k_cache: torch.Tensor, v_cache: torch.Tensor, start: int, *,
                       q_norm_weight: torch.Tensor | None = None, k_norm_weight: torch.Tensor | None = None,
                       theta: float = 1e6, eps: float = RMS_EPS) -> torch.Tensor:
    """Prefill chunk prologue: q/k per-head RMSNorm + RoPE at positions start.., q -> q_out bf16 [n, nh, 128],
    k/v -> bf16 rows of one layer's cache [s_cap, nk, 128].  q, k, v fp32 [n, heads * 128] with unit column
    stride (row views of one wider buffer are fine).

    With caches of shape [n_seq, s_cap, nk, 128], the rows of q, k, v and q_out are n_seq sequences of
    n / n_seq tokens each, every one at positions start.. of its own cache, in one launch."""
    n = int(q.shape[0])
    for t, name in ((q, "q"), (k, "k"), (v, "v")):
        _check_strided(t, name, torch.float32)
        if t.dim() != 2 or t.shape[0] != n or t.shape[1] % 128:
            raise ValueError(f"{name} must be fp32 [n, heads * 128], got {tuple(t.shape)}")
    nh, nk = q.shape[1] // 128, k.shape[1] // 128
    if v.shape[1] != k.shape[1]:
        raise ValueError("k and v must have the same width")
    _check(q_out, "q_out", torch.bfloat16)
    if q_out.numel() != n * nh * 128:
        raise ValueError(f"q_out must hold [{n}, {nh}, 128]")
    if k_cache.dim() == 4:
        n_seq = int(k_cache.shape[0])
        if n_seq == 0 or n % n_seq:
            raise ValueError(f"{n} rows do not split into {n_seq} sequences")
    else:
        n_seq = 1
    for t, name in ((k_cache, "k_cache"), (v_cache, "v_cache")):
        _check(t, name, torch.bfloat16)
        if t.dim() != k_cache.dim() or t.dim() not in (3, 4) or t.shape[-2] != nk or t.shape[-1] != 128 or \
                (t.dim() == 4 and t.shape[0] != n_seq):
            raise ValueError(f"{name} must be bf16 [s_cap, {nk}, 128] or [n_seq, s_cap, {nk}, 128], "
                             f"got {tuple(t.shape)}")
    if v_cache.shape != k_cache.shape:
        raise ValueError("k_cache and v_cache must have the same shape")
    if (q_norm_weight is None) != (k_norm_weight is None):
        raise ValueError("pass both q and k norm weights or neither")
    for t, name in ((q_norm_weight, "q_norm_weight"), (k_norm_weight, "k_norm_weight")):
        if t is not None:
            _check(t, name, torch.float32, align=4)
            if t.numel() != 128:
                raise ValueError(f"{name} must have 128 elements")
    s_cap = int(k_cache.shape[-3])
    per_seq = n // n_seq
    if start < 0 or start + per_seq > s_cap:
        raise ValueError(f"positions {start}..{start + per_seq - 1} exceed the cache capacity {s_cap}")
    head = (ptr(q), q.stride(0), ptr(k), k.stride(0), ptr(v), v.stride(0), ptr(q_norm_weight), ptr(k_norm_weight),
            eps, theta, int(start), per_seq)
    tail = (nh, nk, 128, ptr(q_out), ptr(k_cache), ptr(v_cache), s_cap, stream_handle())
    if k_cache.dim() == 3:
        call("t2h_qk_norm_rope_cache", *head, *tail)
    else:
        call("t2h_qk_norm_rope_cache_seqs", *head, n_seq, *tail)
    return q_out


ACTS = {None: 0, "none": 0, "gelu": 1}


def q8_0_linear(x: torch.Tensor, w: torch.Tensor, *, bias: torch.Tensor | None = None, act: str | None = None,
                out: torch.Tensor | None = None, out_dtype: torch.dtype = torch.bfloat16,
                residual: torch.Tensor | None = None, splits: int | None = None) -> torch.Tensor:
    """y[M, N] = act(x[M, K] . deq(W)^T + bias) (+ residual) on the matrix cores (LINEAR_BIAS_Q8_0W_F32B_F32).
    x bf16 with K % 64 == 0; W Q8_0 rows of w_k = 32 * blocks <= K values (x's columns past w_k must be
    finite: they multiply zeros); bias fp32 [N]; act None or "gelu" (erf by Abramowitz-Stegun 7.1.26, as the
    reference).  From DEQUANT_FIRST_ROWS rows with w_k == K, W is dequantised once and the bf16 rows run
    t2h_bf16_linear (the same bits)."""
    _check(x, "x", torch.bfloat16)
    _check(w, "weight", torch.uint8, align=1)
    k = int(x.shape[-1])
    if k % 64:
        raise ValueError(f"q8_0_linear needs K % 64 == 0 (pad the rows with zeros), got {k}")
    if w.dim() != 2 or w.shape[1] % Q8_0_BYTES or w.shape[1] == 0:
        raise ValueError(f"weight must be uint8 [N, 34 * blocks], got {tuple(w.shape)}")
    w_k = int(w.shape[1]) // Q8_0_BYTES * 32
    if w_k > k:
        raise ValueError(f"weight rows hold {w_k} values, more than x's {k} columns")
    if w.data_ptr() % 2:
        raise ValueError("weight must be 2-byte aligned")
    if act not in ACTS:
        raise ValueError(f"act must be one of {sorted(a for a in ACTS if a)} or None, got {act!r}")
    m = x.numel() // k
    n = int(w.shape[0])
    if bias is not None:
        _check(bias, "bias", torch.float32, align=4)
        if bias.numel() != n:
            raise ValueError(f"bias must have {n} elements, got {bias.numel()}")
    if out is None:
        out = torch.empty(*x.shape[:-1], n, dtype=out_dtype, device=x.device)
    _check(out, "output", tuple(_OUT_DTYPES), align=4)
    if out.numel() != m * n:
        raise ValueError(f"output has {out.numel()} elements, expected {m * n}")
    if residual is not None:
        _check(residual, "residual", torch.float32, align=4)
        if residual.numel() != m * n or out.dtype != torch.float32:
            raise ValueError("residual must be fp32 with the output's shape; output must be fp32")
    splits = gemm_splits(m, n, k) if splits is None else splits
    if splits > 1:
        _gemm_splitk("q8_0", x, w, None, out, m, k, n, w_k, splits, bias=bias, act=ACTS[act], residual=residual)
        return out
    if w_k == k and _dequant_first(m, "q8_0", splits):
        wb = dequantize_bf16(w, "q8_0", k)
        call("t2h_bf16_linear", ptr(x), ptr(wb), ptr(bias), ACTS[act], ptr(out), _OUT_DTYPES[out.dtype], ptr(residual),
             m, k, n, stream_handle())
        return out
    call("t2h_q8_0_linear", ptr(x), ptr(w), ptr(bias), ACTS[act], ptr(out), _OUT_DTYPES[out.dtype], ptr(residual),
         m, k, n, w_k, stream_handle())
    return out


def set_gemv_max_blocks(max_blocks: int, max_blocks_norm: int = 0) -> None:
    """Grid caps (blocks of 8 waves) for plain and RMSNorm-prologue Q4_K GEMV launches."""
    call("t2h_set_gemv_max_blocks", int(max_blocks), int(max_blocks_norm))


# ------------------------------------------------------- token selection --


def token_select(partial_scores: torch.Tensor, partial_tokens: torch.Tensor, eos_ids: torch.Tensor,
                 next_token: torch.Tensor, done: torch.Tensor) -> None:
    _check(partial_scores, "scores", torch.float32, align=4)
    _check(partial_tokens, "tokens", _TOKEN_DTYPES, align=4)
    _check(eos_ids, "eos_token_ids", torch.int64, align=8)
    _check(next_token, "next_token", torch.int64, align=8)
    _check(done, "done", _TOKEN_DTYPES, align=4)
    call("t2h_token_select", ptr(partial_scores), ptr(partial_tokens), partial_scores.numel(), ptr(eos_ids),
         eos_ids.numel(), ptr(next_token), ptr(done), stream_handle())


def token_store(next_token: torch.Tensor, done: torch.Tensor, generated: torch.Tensor, length: torch.Tensor,
                stopped: torch.Tensor, *, stop_on_eos: bool = True, token_index: int = 0,
                token_index_ptr: torch.Tensor | None = None, advance: torch.Tensor | None = None) -> None:
    _check(next_token, "next_token", torch.int64, align=8)
    _check(done, "done", _TOKEN_DTYPES, align=4)
    _check(generated, "generated_tokens", torch.int64, align=8)
    _check(length, "generated_length", _TOKEN_DTYPES, align=4)
    _check(stopped, "stopped", _TOKEN_DTYPES, align=4)
    if token_index_ptr is not None:
        _check(token_index_ptr, "token_index", torch.int32, align=4)
    if advance is not None:
        _check(advance, "advance", torch.int32, align=4)
    call("t2h_token_store", ptr(next_token), ptr(done), ptr(generated), generated.numel(), ptr(length),
         ptr(stopped), int(stop_on_eos), ptr(token_index_ptr), int(token_index), ptr(advance), stream_handle())


def token_select_store(partial_scores: torch.Tensor, partial_tokens: torch.Tensor, eos_ids: torch.Tensor,
                       next_token: torch.Tensor, done: torch.Tensor, generated: torch.Tensor, length: torch.Tensor,
                       stopped: torch.Tensor, *, stop_on_eos: bool = True, advance: torch.Tensor | None = None) -> None:
    """token_select + token_store (index from the device length counter) in one launch."""
    _check(partial_scores, "scores", torch.float32, align=4)
    _check(partial_tokens, "tokens", _TOKEN_DTYPES, align=4)
    _check(eos_ids, "eos_token_ids", torch.int64, align=8)
    _check(next_token, "next_token", torch.int64, align=8)
    _check(done, "done", _TOKEN_DTYPES, align=4)
    _check(generated, "generated_tokens", torch.int64, align=8)
    _check(length, "generated_length", _TOKEN_DTYPES, align=4)
    _check(stopped, "stopped", _TOKEN_DTYPES, align=4)
    if advance is not None:
        _check(advance, "advance", torch.int32, align=4)
    call("t2h_token_select_store", ptr(partial_scores), ptr(partial_tokens), partial_scores.numel(), ptr(eos_ids),
         eos_ids.numel(), ptr(next_token), ptr(done), ptr(generated), generated.numel(), ptr(length), ptr(stopped),
         int(stop_on_eos), ptr(advance), stream_handle())



def _tensor_ptrs(ts: list[torch.Tensor | None]):
    """A ctypes array of the tensors' device addresses (null for None), kept alive by the caller."""
    return (ctypes.c_void_p * len(ts))(*[None if t is None else t.data_ptr() for t in ts])


def token_select_store_seqs(partial_scores: list[torch.Tensor], partial_tokens: list[torch.Tensor],
                            eos_ids: torch.Tensor, next_tokens: list[torch.Tensor], dones: list[torch.Tensor],
                            generated: list[torch.Tensor], lengths: list[torch.Tensor], stopped: list[torch.Tensor],
                            *, stop_on_eos: bool = True, advance: list[torch.Tensor] | None = None) -> None:
    """token_select_store of 1..4 sequences in one launch (t2h_token_select_store_seqs); argument i of every
    list belongs to sequence i, and each sequence's result equals its own call."""
    n = len(partial_scores)
    lists = (partial_tokens, next_tokens, dones, generated, lengths, stopped) + ((advance,) if advance else ())
    if not 1 <= n <= LM_HEAD_SEQS_MAX or any(len(x) != n for x in lists):
        raise ValueError(f"1..{LM_HEAD_SEQS_MAX} sequences with one of each argument per sequence")
    g, cap = partial_scores[0].numel(), generated[0].numel()
    _check(eos_ids, "eos_token_ids", torch.int64, align=8)
    for i in range(n):
        _check(partial_scores[i], "scores", torch.float32, align=4)
        _check(partial_tokens[i], "tokens", _TOKEN_DTYPES, align=4)
        _check(next_tokens[i], "next_token", torch.int64, align=8)
        _check(dones[i], "done", _TOKEN_DTYPES, align=4)
        _check(generated[i], "generated_tokens", torch.int64, align=8)
        _check(lengths[i], "generated_length", _TOKEN_DTYPES, align=4)
        _check(stopped[i], "stopped", _TOKEN_DTYPES, align=4)
        if advance:
            _check(advance[i], "advance", torch.int32, align=4)
        if partial_scores[i].numel() != g or partial_tokens[i].numel() != g or generated[i].numel() != cap:
            raise ValueError("every sequence needs the same partial count and generated capacity")
    arrs = [_tensor_ptrs(x) for x in (partial_scores, partial_tokens, next_tokens, dones, generated, lengths, stopped,
                                    advance if advance else [None] * n)]
    sc, tk, nt, dn, gen, ln, st, adv = (ctypes.addressof(a) for a in arrs)
    call("t2h_token_select_store_seqs", n, sc, tk, g, ptr(eos_ids), eos_ids.numel(), nt, dn, gen, cap, ln, st,
         int(stop_on_eos), adv, stream_handle())


# ------------------------------------------------------ decode attention --


def attn_decode_workspace_bytes(nh: int, nk: int, d: int, s_cap: int) -> int:
    n = int(_lib.lib().t2h_attn_decode_workspace_bytes(nh, nk, d, s_cap))
    if n == 0:
        raise ValueError(f"unsupported attention shape nh={nh} nk={nk} d={d}")
    return n


def attn_decode_workspace(nh: int, nk: int, d: int, s_cap: int, device) -> torch.Tensor:
    """Zeroed workspace; the kernel leaves it reusable across calls."""
    return torch.zeros(attn_decode_workspace_bytes(nh, nk, d, s_cap), dtype=torch.uint8, device=device)


def attn_decode(q: torch.Tensor, k_new: torch.Tensor, v_new: torch.Tensor, k_cache: torch.Tensor,
                v_cache: torch.Tensor, out: torch.Tensor, cache_position: torch.Tensor, workspace: torch.Tensor, *,
                q_norm_weight: torch.Tensor | None = None, k_norm_weight: torch.Tensor | None = None,
                theta: float = 0.0, eps: float = RMS_EPS) -> torch.Tensor:
    """One-token split-K attention; q [NH, D], k_new/v_new [NK, D] fp32; caches bf16 [S, NK, D]."""
    for t, name in ((q, "q"), (k_new, "new_k"), (v_new, "new_v")):
        _check(t, name, torch.float32, align=4)
    _check(k_cache, "k_cache", torch.bfloat16)
    _check(v_cache, "v_cache", torch.bfloat16)
    _check(out, "output", torch.bfloat16, align=4)
    _check(cache_position, "cache_position", torch.int32, align=4)
    _check(workspace, "workspace", torch.uint8)
    if k_cache.dim() != 3 or v_cache.shape != k_cache.shape:
        raise ValueError("k_cache/v_cache must both be [S, NK, D]")
    s_cap, nk, d = k_cache.shape
    nh = q.numel() // d
    if q.numel() != nh * d or k_new.numel() != nk * d or v_new.numel() != nk * d or out.numel() != nh * d:
        raise ValueError("q/new_k/new_v/output sizes do not match the cache's NK and D")
    for t, name in ((q_norm_weight, "q_norm"), (k_norm_weight, "k_norm")):
        if t is not None:
            _check(t, name, torch.float32, align=4)
            if t.numel() != d:
                raise ValueError(f"{name} weight must have D elements")
    call("t2h_attn_decode", ptr(q), ptr(k_new), ptr(v_new), ptr(q_norm_weight), ptr(k_norm_weight), eps, theta,
         ptr(k_cache), ptr(v_cache), ptr(out), nh, nk, d, s_cap, ptr(cache_position), ptr(workspace),
         workspace.numel(), stream_handle())
    return out


# ------------------------------------------------ persistent decode layers --

DECODE_LAYER_FIELDS = ("q", "k", "v", "o", "gate", "up", "down", "input_norm", "post_norm", "q_norm", "k_norm")


def decode_layers_supported(hidden: int, mlp: int, nh: int, nk: int, d: int) -> bool:
    return int(_lib.lib().t2h_qwen3_decode_layers_workspace_bytes(hidden, mlp, nh, nk, d)) > 0


def decode_layers_workspace(hidden: int, mlp: int, nh: int, nk: int, d: int, device) -> torch.Tensor | None:
    """Zeroed workspace of the persistent decode kernel, or None when the shape is not built."""
    n = int(_lib.lib().t2h_qwen3_decode_layers_workspace_bytes(hidden, mlp, nh, nk, d))
    return torch.zeros(n, dtype=torch.uint8, device=device) if n else None


DECODE_LAYER_TABLE_COLUMNS = 14
DL_WT_V_Q6, DL_WT_DOWN_Q6 = 1, 2  # bits of the table's weight-types column


def decode_layer_table(packed: dict[str, torch.Tensor], norms: dict[str, torch.Tensor], layers: int,
                       k_cache: torch.Tensor, v_cache: torch.Tensor,
                       types: dict[str, str] | None = None) -> torch.Tensor:
    """Device int64 [layers, 14] table for :func:`decode_layers`: the q, k, v, o, gate, up, down, norm and cache
    pointers, then the layer's weight types (bit 0: v is Q6_K, bit 1: down is Q6_K).  ``types`` (GGUF type per
    weight name; None = all Q4_K): q, k, o, gate and up must be Q4_K, v and down Q4_K or Q6_K (the Q4_K_M
    policy).  q and k must be consecutive rows of one allocation, followed by v's rows when v is Q4_K."""
    rows = []
    for i in range(layers):
        p = f"layers.{i}."
        t = {n: (types[p + n] if types is not None else "q4_k") for n in ("q", "k", "v", "o", "gate", "up", "down")}
        for n in ("q", "k", "o", "gate", "up"):
            if t[n] != "q4_k":
                raise ValueError(f"layer {i}: {n} must be Q4_K, got {t[n]}")
        for n in ("v", "down"):
            if t[n] not in ("q4_k", "q6_k"):
                raise ValueError(f"layer {i}: {n} must be Q4_K or Q6_K, got {t[n]}")
        q, k, v = packed[p + "q"], packed[p + "k"], packed[p + "v"]
        if k.data_ptr() != q.data_ptr() + q.numel():
            raise ValueError(f"layer {i}: q and k rows must be stacked in one allocation")
        if t["v"] == "q4_k" and v.data_ptr() != k.data_ptr() + k.numel():
            raise ValueError(f"layer {i}: a Q4_K v must follow k's rows in the same allocation")
        ptrs = [packed[p + n].data_ptr() for n in ("q", "k", "v", "o", "gate", "up", "down")]
        ptrs += [norms[p + n].data_ptr() for n in ("input_norm", "post_norm", "q_norm", "k_norm")]
        ptrs += [k_cache[i].data_ptr(), v_cache[i].data_ptr()]
        ptrs.append((DL_WT_V_Q6 if t["v"] == "q6_k" else 0) | (DL_WT_DOWN_Q6 if t["down"] == "q6_k" else 0))
        rows.append(ptrs)
    return torch.tensor(rows, dtype=torch.int64).to(k_cache.device)


def decode_layers(table: torch.Tensor, h: torch.Tensor, cache_position: torch.Tensor, workspace: torch.Tensor,
                  status: torch.Tensor, *, hidden: int, mlp: int, nh: int, nk: int, d: int, s_cap: int,
                  eps: float = RMS_EPS, theta: float = 1.0e6, trace: torch.Tensor | None = None) -> None:
    """All decoder layers of one token in one persistent launch (h updated in place).  ``trace`` (uint64
    [layers, 6, 256, 8], see decode_layers_trace) runs the instantiation that records the phase timeline."""
    _check(table, "layer_table", torch.int64, align=8)
    _check(h, "h", torch.float32)
    _check(cache_position, "cache_position", torch.int32, align=4)
    _check(workspace, "workspace", torch.uint8, align=256)
    _check(status, "status", torch.int32, align=4)
    if table.dim() != 2 or table.shape[1] != DECODE_LAYER_TABLE_COLUMNS:
        raise ValueError(f"layer_table must be int64 [layers, {DECODE_LAYER_TABLE_COLUMNS}], got {tuple(table.shape)}")
    args = (ptr(table), int(table.shape[0]), hidden, mlp, nh, nk, d, s_cap, ptr(h), ptr(cache_position), eps, theta,
            ptr(workspace), workspace.numel(), ptr(status))
    if trace is None:
        call("t2h_qwen3_decode_layers", *args, stream_handle())
    else:
        _check(trace, "trace", torch.int64, align=8)
        call("t2h_qwen3_decode_layers_traced", *args, ptr(trace), trace.numel() * 8, stream_handle())


def decode_layers_noalloc(table: torch.Tensor, h: torch.Tensor, cache_position: torch.Tensor, status: torch.Tensor,
                          *, hidden: int, mlp: int, nh: int, nk: int, d: int, s_cap: int, eps: float = RMS_EPS,
                          theta: float = 1.0e6) -> None:
    """decode_layers with the library's own per-GPU workspace (t2h_qwen3_decode_layers_noalloc): no device memory is
    allocated, by the library or here.  Calls on one GPU must not overlap."""
    _check(table, "layer_table", torch.int64, align=8)
    _check(h, "h", torch.float32)
    _check(cache_position, "cache_position", torch.int32, align=4)
    _check(status, "status", torch.int32, align=4)
    if table.dim() != 2 or table.shape[1] != DECODE_LAYER_TABLE_COLUMNS:
        raise ValueError(f"layer_table must be int64 [layers, {DECODE_LAYER_TABLE_COLUMNS}], got {tuple(table.shape)}")
    call("t2h_qwen3_decode_layers_noalloc", ptr(table), int(table.shape[0]), hidden, mlp, nh, nk, d, s_cap, ptr(h),
         ptr(cache_position), eps, theta, ptr(status), stream_handle())


DECODE_SEQS = (1, 4)  # sequences one persistent launch can run (4: the Qwen3-0.6B shape, s_cap <= 2048)
LM_HEAD_SEQS_MAX = 4  # sequences of one t2h_q4k_lm_head_argmax_partial_seqs launch


def decode_layers_seqs(tables: list[torch.Tensor], hs: list[torch.Tensor], cache_positions: list[torch.Tensor],
                       workspaces: list[torch.Tensor], statuses: list[torch.Tensor], *, hidden: int, mlp: int,
                       nh: int, nk: int, d: int, s_cap: int, eps: float = RMS_EPS, theta: float = 1.0e6,
                       trace: torch.Tensor | None = None) -> None:
    """decode_layers for len(tables) sequences in one persistent launch (t2h_qwen3_decode_layers_seqs): each
    sequence its own table (its KV caches), h, position, workspace and status.  ``trace`` (decode_layers_trace)
    records the launch's phase timeline, sequence i in blocks 256 i / n .. 256 (i + 1) / n - 1."""
    n = len(tables)
    if n not in DECODE_SEQS or not (len(hs) == len(cache_positions) == len(workspaces) == len(statuses) == n):
        raise ValueError(f"decode_layers_seqs runs {DECODE_SEQS} sequences with one of each argument per sequence")
    for i in range(n):
        _check(tables[i], "layer_table", torch.int64, align=8)
        _check(hs[i], "h", torch.float32)
        _check(cache_positions[i], "cache_position", torch.int32, align=4)
        _check(workspaces[i], "workspace", torch.uint8, align=256)
        _check(statuses[i], "status", torch.int32, align=4)
        if tables[i].dim() != 2 or tables[i].shape != tables[0].shape or tables[i].shape[1] != DECODE_LAYER_TABLE_COLUMNS:
            raise ValueError("layer tables must all be int64 [layers, 14]")
        if workspaces[i].numel() != workspaces[0].numel():
            raise ValueError("workspaces must all have the same size")
    if len({w.data_ptr() for w in workspaces}) != n:
        raise ValueError("every sequence needs its own workspace")
    arr = lambda ts: (ctypes.c_void_p * n)(*[t.data_ptr() for t in ts])  # noqa: E731
    t_arr, h_arr, p_arr, w_arr, s_arr = arr(tables), arr(hs), arr(cache_positions), arr(workspaces), arr(statuses)
    args = (n, ctypes.addressof(t_arr), int(tables[0].shape[0]), hidden, mlp, nh, nk, d, s_cap,
            ctypes.addressof(h_arr), ctypes.addressof(p_arr), eps, theta, ctypes.addressof(w_arr),
            workspaces[0].numel(), ctypes.addressof(s_arr))
    if trace is None:
        call("t2h_qwen3_decode_layers_seqs", *args, stream_handle())
    else:
        _check(trace, "trace", torch.int64, align=8)
        call("t2h_qwen3_decode_layers_seqs_traced", *args, ptr(trace), trace.numel() * 8, stream_handle())


DECODE_TRACE_PHASES = ("qkv", "attention", "merge", "o", "gate_up", "down")
DECODE_TRACE_SLOTS = ("begin", "ready", "first", "end", "polls")


def decode_layers_trace(layers: int, device) -> torch.Tensor:
    """Buffer for the persistent kernel's phase timeline: int64 [layers, 6 phases, 256 blocks, 8 slots]; slots
    0-3 are 100 MHz clock stamps (DECODE_TRACE_SLOTS), slot 4 a poll count."""
    shape = (layers, len(DECODE_TRACE_PHASES), 256, 8)
    if int(_lib.lib().t2h_qwen3_decode_layers_trace_bytes(layers)) != 8 * layers * 6 * 256 * 8:
        raise RuntimeError("libt2h's trace layout differs from this wrapper's")
    return torch.zeros(shape, dtype=torch.int64, device=device)


# ------------------------------------------------------ prefill attention --


def _check_strided(t: torch.Tensor, name: str, dtype: torch.dtype) -> None:
    """Device, dtype and a contiguous last dimension; other strides are free (the kernel takes them)."""
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor, got {type(t).__name__}")
    if t.device.type != "cuda":
        raise ValueError(f"{name} must live on a HIP device, got {t.device}")
    if t.dtype != dtype:
        raise TypeError(f"{name} dtype {t.dtype}, expected {dtype}")
    if t.stride(-1) != 1:
        raise ValueError(f"{name} needs a contiguous last dimension")


FA_BLOCK_QUERIES = 128  # queries per flash-attention block (a row of mask tiles)
FA_TILE_KEYS = 64       # keys per flash-attention tile


def fa_mask_tiles(mask: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """uint8 [B, ceil(T/128), ceil(S/64)] class of each 128 x 64 block of an additive fp32 mask [B, T, S]:
    1 all masked (every entry <= -FLT_MAX/2), 2 all zero, 0 mixed (the reference's FA_MASK_OPT_F16 rule).  A mask
    used by several attention calls (every layer of one pass) is classified once."""
    _check_strided(mask, "mask", torch.float32)
    if mask.dim() != 3:
        raise ValueError(f"mask must be rank 3 [B, T, S], got {tuple(mask.shape)}")
    b, t_len, s_len = mask.shape
    want = (b, -(-t_len // FA_BLOCK_QUERIES), -(-s_len // FA_TILE_KEYS))
    tiles = torch.empty(want, dtype=torch.uint8, device=mask.device) if out is None else out
    _check(tiles, "mask_tiles", torch.uint8, align=1)
    if tuple(tiles.shape) != want:
        raise ValueError(f"mask_tiles must be {want}, got {tuple(tiles.shape)}")
    call("t2h_fa_mask_tiles", ptr(mask), b, t_len, s_len, mask.stride(0), mask.stride(1), ptr(tiles),
         stream_handle())
    return tiles


def flash_attn_prefill(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, out: torch.Tensor | None = None, *,
                       causal: bool = True, causal_offset: int = 0, mask: torch.Tensor | None = None,
                       scale: float | None = None, mask_tiles: torch.Tensor | bool | None = None) -> torch.Tensor:
    """softmax(q k^T * scale + mask) v; q/out [B, T, NH, D], k/v [B, S, NK, D], bf16, any (batch, token, head)
    strides with D contiguous -- token-major tensors as they are, head-major ones as ``x.transpose(1, 2)``.
    ``mask``: additive fp32 [B or 1, T, S] (S contiguous).  Causal: query t sees keys <= t + causal_offset.
    ``mask_tiles``: the mask's fa_mask_tiles (computed here when None; False reads every mask entry): all-masked
    tiles are skipped and all-zero tiles not read -- the same result, except that a query whose every key is
    masked gets zeros."""
    for t, name in ((q, "q"), (k, "k"), (v, "v")):
        _check_strided(t, name, torch.bfloat16)
        if t.dim() != 4:
            raise ValueError(f"{name} must be rank 4 [B, T, H, D], got {tuple(t.shape)}")
    b, t_len, nh, d = q.shape
    _, s_len, nk, _ = k.shape
    if k.shape[0] != b or v.shape != k.shape or k.shape[3] != d:
        raise ValueError(f"shape mismatch q {tuple(q.shape)} k {tuple(k.shape)} v {tuple(v.shape)}")
    if out is None:
        out = torch.empty(b, t_len, nh, d, dtype=torch.bfloat16, device=q.device)
    _check_strided(out, "output", torch.bfloat16)
    if tuple(out.shape) != (b, t_len, nh, d):
        raise ValueError(f"output must be {(b, t_len, nh, d)}, got {tuple(out.shape)}")
    m_sb = m_st = 0
    if mask is not None:
        _check_strided(mask, "mask", torch.float32)
        if mask.dim() != 3 or mask.shape[1] != t_len or mask.shape[2] != s_len or mask.shape[0] not in (1, b):
            raise ValueError(f"mask must be [B or 1, {t_len}, {s_len}], got {tuple(mask.shape)}")
        m_sb = mask.stride(0) if mask.shape[0] == b else 0
        m_st = mask.stride(1)
    strides = (_lib.ctypes.c_int64 * 14)(q.stride(0), q.stride(1), q.stride(2), k.stride(0), k.stride(1),
                                         k.stride(2), v.stride(0), v.stride(1), v.stride(2), out.stride(0),
                                         out.stride(1), out.stride(2), m_sb, m_st)
    if mask is not None and mask_tiles is not False:
        tiles = fa_mask_tiles(mask) if mask_tiles is None or mask_tiles is True else mask_tiles
        want = (mask.shape[0], -(-t_len // FA_BLOCK_QUERIES), -(-s_len // FA_TILE_KEYS))
        _check(tiles, "mask_tiles", torch.uint8, align=1)
        if tuple(tiles.shape) != want:
            raise ValueError(f"mask_tiles must be {want} (fa_mask_tiles of the mask), got {tuple(tiles.shape)}")
        call("t2h_flash_attn_prefill_tiles", ptr(q), ptr(k), ptr(v), ptr(out), ptr(mask), ptr(tiles), b, nh, nk,
             t_len, s_len, d, strides, 1 if causal else 0, int(causal_offset), float(scale or 0.0), stream_handle())
        return out
    call("t2h_flash_attn_prefill", ptr(q), ptr(k), ptr(v), ptr(out), ptr(mask), b, nh, nk, t_len, s_len, d,
         strides, 1 if causal else 0, int(causal_offset), float(scale or 0.0), stream_handle())
    return out


def segment_bounds(cu_seqlens, t_len: int, device) -> torch.Tensor:
    """Validated int32 segment bounds on the device: ascending, cu[0] == 0, cu[-1] == t_len.  A device tensor
    is taken as it is (the kernel clamps every key range, so a bad table gives wrong windows, never a fault)."""
    if isinstance(cu_seqlens, torch.Tensor) and cu_seqlens.device.type == "cuda":
        _check(cu_seqlens, "cu_seqlens", torch.int32, align=4)
        return cu_seqlens
    cu = torch.as_tensor(cu_seqlens, dtype=torch.int64).reshape(-1)
    if cu.numel() < 2 or int(cu[0]) != 0 or int(cu[-1]) != t_len or bool((cu[1:] < cu[:-1]).any()):
        raise ValueError(f"cu_seqlens must ascend from 0 to {t_len}, got {cu.tolist()[:8]}...")
    return cu.to(device=device, dtype=torch.int32)


def flash_attn_segments(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cu_seqlens, out: torch.Tensor | None = None,
                        *, scale: float | None = None) -> torch.Tensor:
    """Self-attention within segments: token t attends to the tokens of its own segment [cu[i], cu[i+1]).
    q/out [B, T, NH, D], k/v [B, T, NK, D] bf16 with D contiguous (any other strides).  Equals SDPA_MASKED_F32
    under the block-diagonal window mask of the Qwen3-ASR encoder, without the mask."""
    for t, name in ((q, "q"), (k, "k"), (v, "v")):
        _check_strided(t, name, torch.bfloat16)
        if t.dim() != 4:
            raise ValueError(f"{name} must be rank 4 [B, T, H, D], got {tuple(t.shape)}")
    b, t_len, nh, d = q.shape
    nk = k.shape[2]
    if k.shape[0] != b or k.shape[1] != t_len or v.shape != k.shape or k.shape[3] != d:
        raise ValueError(f"shape mismatch q {tuple(q.shape)} k {tuple(k.shape)} v {tuple(v.shape)}")
    cu = segment_bounds(cu_seqlens, t_len, q.device)
    if out is None:
        out = torch.empty(b, t_len, nh, d, dtype=torch.bfloat16, device=q.device)
    _check_strided(out, "output", torch.bfloat16)
    if tuple(out.shape) != (b, t_len, nh, d):
        raise ValueError(f"output must be {(b, t_len, nh, d)}, got {tuple(out.shape)}")
    strides = (_lib.ctypes.c_int64 * 12)(q.stride(0), q.stride(1), q.stride(2), k.stride(0), k.stride(1),
                                         k.stride(2), v.stride(0), v.stride(1), v.stride(2), out.stride(0),
                                         out.stride(1), out.stride(2))
    call("t2h_flash_attn_segments", ptr(q), ptr(k), ptr(v), ptr(out), ptr(cu), cu.numel() - 1, b, nh, nk, t_len, d,
         strides, float(scale or 0.0), stream_handle())
    return out


# -------------------------------------------------------------- small ops --


def embedding_q4_k(w: torch.Tensor, ids: torch.Tensor, dim: int, out: torch.Tensor | None = None) -> torch.Tensor:
    _check(w, "weight", torch.uint8)  # 16-byte superblock loads
    _check(ids, "indices", torch.int64, align=8)
    if w.shape[1] != q4_k_row_bytes(dim):
        raise ValueError("embedding weight width does not match dim")
    if out is None:
        out = torch.empty(ids.numel(), dim, dtype=torch.float32, device=w.device)
    _check(out, "output", torch.float32)  # float4 stores
    call("t2h_embedding_q4_k", ptr(w), int(w.shape[0]), ptr(ids), ids.numel(), dim, ptr(out), stream_handle())
    return out


def embedding_q4_k_seqs(w: torch.Tensor, ids: list[torch.Tensor], dim: int, outs: list[torch.Tensor]) -> None:
    """One token of each of 1..4 sequences (ids[i][0]) embedded into outs[i] (fp32 [dim]) in one launch
    (t2h_embedding_q4_k_seqs)."""
    n = len(ids)
    if not 1 <= n <= LM_HEAD_SEQS_MAX or len(outs) != n:
        raise ValueError(f"1..{LM_HEAD_SEQS_MAX} sequences with one id tensor and one output each")
    _check(w, "weight", torch.uint8, align=1)
    if w.shape[1] != q4_k_row_bytes(dim):
        raise ValueError("embedding weight width does not match dim")
    for i in range(n):
        _check(ids[i], "indices", torch.int64, align=8)
        _check(outs[i], "output", torch.float32, align=16)
        if ids[i].numel() < 1 or outs[i].numel() != dim:
            raise ValueError("each sequence needs one id and a [dim] output")
    id_arr, out_arr = _tensor_ptrs(ids), _tensor_ptrs(outs)
    call("t2h_embedding_q4_k_seqs", n, ptr(w), int(w.shape[0]), ctypes.addressof(id_arr), dim,
         ctypes.addressof(out_arr), stream_handle())


def rms_norm(x: torch.Tensor, weight: torch.Tensor, out: torch.Tensor | None = None,
             eps: float = RMS_EPS) -> torch.Tensor:
    _check(x, "x", tuple(_OUT_DTYPES), align=2)
    _check(weight, "weight", torch.float32, align=4)
    h = int(x.shape[-1])
    if weight.numel() != h:
        raise ValueError("weight must have H elements")
    if out is None:
        out = torch.empty_like(x)
    _check(out, "output", tuple(_OUT_DTYPES), align=2)
    call("t2h_rms_norm", ptr(x), _OUT_DTYPES[x.dtype], ptr(weight), ptr(out), _OUT_DTYPES[out.dtype],
         x.numel() // h, h, eps, stream_handle())
    return out


def swiglu(gate: torch.Tensor, up: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    _check(gate, "gate", tuple(_OUT_DTYPES), align=2)
    _check(up, "up", gate.dtype, align=2)
    if up.shape != gate.shape:
        raise ValueError("gate and up must have the same shape")
    if out is None:
        out = torch.empty(gate.shape, dtype=torch.bfloat16, device=gate.device)
    _check(out, "output", torch.bfloat16, align=2)
    call("t2h_swiglu", ptr(gate), ptr(up), _OUT_DTYPES[gate.dtype], ptr(out), gate.numel(), stream_handle())
    return out


# ------------------------------------------------- Qwen3-ASR audio tower --

_IN_DTYPES = {torch.float32: T2H_DTYPE_F32, torch.bfloat16: T2H_DTYPE_BF16}


def conv_out_size(size: int, kernel: int, stride: int, pad: int) -> int:
    return (size + 2 * pad - kernel) // stride + 1


def im2col(x: torch.Tensor, kernel: tuple[int, int], stride: tuple[int, int] = (1, 1),
           padding: tuple[int, int] = (0, 0), *, out_cols: int | None = None,
           out: torch.Tensor | None = None) -> torch.Tensor:
    """Patch rows of a conv2d: x [B, C, H, W] fp32 or bf16 with any strides (a channels-last buffer is passed
    as its permuted view) -> bf16 [B * Ho * Wo, out_cols], column (c, fh, fw) as in F.unfold; the columns past
    C * kh * kw are zero (out_cols defaults to that count rounded up to 64, the GEMM's K step)."""
    if not isinstance(x, torch.Tensor) or x.device.type != "cuda":
        raise ValueError("x must be a tensor on a HIP device")
    if x.dtype not in _IN_DTYPES:
        raise TypeError(f"x dtype {x.dtype} not in {tuple(_IN_DTYPES)}")
    if x.dim() != 4:
        raise ValueError(f"x must be [B, C, H, W], got {tuple(x.shape)}")
    b, c, h, w_ = (int(d) for d in x.shape)
    kh, kw = kernel
    sh, sw = stride
    ph, pw = padding
    ho, wo = conv_out_size(h, kh, sh, ph), conv_out_size(w_, kw, sw, pw)
    if ho <= 0 or wo <= 0:
        raise ValueError(f"kernel {kernel} does not fit input {(h, w_)} with padding {padding}")
    cols = c * kh * kw
    if out_cols is None:
        out_cols = -(-cols // 64) * 64
    if out_cols < cols:
        raise ValueError(f"out_cols {out_cols} < C * kh * kw = {cols}")
    rows = b * ho * wo
    if out is None:
        out = torch.empty(rows, out_cols, dtype=torch.bfloat16, device=x.device)
    _check(out, "output", torch.bfloat16, align=2)
    if tuple(out.shape) != (rows, out_cols):
        raise ValueError(f"output must be {(rows, out_cols)}, got {tuple(out.shape)}")
    strides = (_lib.ctypes.c_int64 * 4)(*(int(st) for st in x.stride()))
    call("t2h_im2col", ptr(x), _IN_DTYPES[x.dtype], strides, b, c, h, w_, kh, kw, sh, sw, ph, pw, ho, wo, ptr(out),
         out_cols, stream_handle())
    return out


def layer_norm(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor, out: torch.Tensor | None = None, *,
               out_dtype: torch.dtype = torch.bfloat16, eps: float = 1e-5) -> torch.Tensor:
    """LayerNorm over the last dimension (LAYER_NORM_F32W_F32B_F32); x fp32 or bf16, out fp32 or bf16."""
    _check(x, "x", tuple(_IN_DTYPES))
    cols = int(x.shape[-1])
    for t, name in ((weight, "weight"), (bias, "bias")):
        _check(t, name, torch.float32)
        if t.numel() != cols:
            raise ValueError(f"{name} must have {cols} elements")
    if out is None:
        out = torch.empty(x.shape, dtype=out_dtype, device=x.device)
    _check(out, "output", tuple(_IN_DTYPES))
    if out.numel() != x.numel():
        raise ValueError("output must have x's shape")
    call("t2h_layer_norm", ptr(x), _IN_DTYPES[x.dtype], ptr(weight), ptr(bias), ptr(out), _IN_DTYPES[out.dtype],
         x.numel() // cols, cols, float(eps), stream_handle())
    return out


def gelu(x: torch.Tensor, out: torch.Tensor | None = None, *, out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """x * (1 + erf(x / sqrt 2)) / 2 (GELU_F32); x, out fp32 or bf16, numel % 4 == 0."""
    _check(x, "x", tuple(_IN_DTYPES), align=8)
    if out is None:
        out = torch.empty(x.shape, dtype=out_dtype or x.dtype, device=x.device)
    _check(out, "output", tuple(_IN_DTYPES), align=8)
    if out.numel() != x.numel():
        raise ValueError("output must have x's shape")
    if x.numel() % 4:
        raise ValueError("gelu needs numel % 4 == 0")
    call("t2h_gelu", ptr(x), _IN_DTYPES[x.dtype], ptr(out), _IN_DTYPES[out.dtype], x.numel(), stream_handle())
    return out


def _row_bytes_of(t: torch.Tensor) -> int:
    rb = t[0].numel() * t.element_size() if t.shape[0] else 0
    if rb % 4:
        raise ValueError("rows must be a multiple of 4 bytes")
    return rb


def index_select_rows(src: torch.Tensor, idx: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """out[i] = src[idx[i]] along dim 0 (INDEX_SELECT_F32); an index out of range gives a zero row."""
    _check(src, "src", (torch.float32, torch.bfloat16, torch.int32), align=4)
    _check(idx, "index", torch.int64, align=8)
    if out is None:
        out = torch.empty(idx.numel(), *src.shape[1:], dtype=src.dtype, device=src.device)
    _check(out, "output", src.dtype, align=4)
    if out.shape[0] != idx.numel() or out.shape[1:] != src.shape[1:]:
        raise ValueError("output must be [len(index), *src.shape[1:]]")
    call("t2h_index_select_rows", ptr(src), int(src.shape[0]), _row_bytes_of(src), ptr(idx), idx.numel(), ptr(out),
         stream_handle())
    return out


def index_copy_rows(dst: torch.Tensor, idx: torch.Tensor, src: torch.Tensor) -> torch.Tensor:
    """dst[idx[i]] = src[i] along dim 0, in place (INDEX_COPY_F32, the audio injection); an index out of range
    is skipped."""
    _check(dst, "dst", (torch.float32, torch.bfloat16, torch.int32), align=4)
    _check(src, "src", dst.dtype, align=4)
    _check(idx, "index", torch.int64, align=8)
    if src.shape[0] != idx.numel() or src.shape[1:] != dst.shape[1:]:
        raise ValueError("src must be [len(index), *dst.shape[1:]]")
    call("t2h_index_copy_rows", ptr(dst), int(dst.shape[0]), _row_bytes_of(dst), ptr(idx), idx.numel(), ptr(src),
         stream_handle())
    return dst


def embedding_q8_0(w: torch.Tensor, ids: torch.Tensor, dim: int, out: torch.Tensor | None = None) -> torch.Tensor:
    """fp32 rows of a Q8_0 embedding table (EMBEDDING_Q8_0_F32); an id out of range gives zeros."""
    _check(w, "weight", torch.uint8, align=2)
    _check(ids, "indices", torch.int64, align=8)
    if dim % 32 or w.dim() != 2 or w.shape[1] != dim // 32 * Q8_0_BYTES:
        raise ValueError("embedding weight width does not match dim")
    if out is None:
        out = torch.empty(ids.numel(), dim, dtype=torch.float32, device=w.device)
    _check(out, "output", torch.float32)
    call("t2h_embedding_q8_0", ptr(w), int(w.shape[0]), ptr(ids), ids.numel(), dim, ptr(out), stream_handle())
    return out


SNAKE_EPS = 1e-9  # add_scalar.py:43 of the reference's OmniVoice decoder


def conv1d_out_len(length: int, kernel: int, stride: int = 1, padding: int = 0, dilation: int = 1) -> int:
    return (length + 2 * padding - dilation * (kernel - 1) - 1) // stride + 1


def im2col_1d(x: torch.Tensor, kernel: int, *, stride: int = 1, padding: int = 0, dilation: int = 1,
              out_cols: int | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """conv1d taps of x [B, L, C] (channels-last, fp32 or bf16, any strides) -> bf16 [B * Lo, out_cols], column
    c * K + k = x[b, t * stride + k * dilation - padding, c] (zero outside); columns past C * K are zero
    (out_cols defaults to C * K rounded up to 64, the GEMM's K step)."""
    if not isinstance(x, torch.Tensor) or x.device.type != "cuda":
        raise ValueError("x must be a tensor on a HIP device")
    if x.dtype not in _IN_DTYPES:
        raise TypeError(f"x dtype {x.dtype} not in {tuple(_IN_DTYPES)}")
    if x.dim() != 3:
        raise ValueError(f"x must be [B, L, C], got {tuple(x.shape)}")
    b, length, c = (int(d) for d in x.shape)
    lo = conv1d_out_len(length, kernel, stride, padding, dilation)
    if lo < 1:
        raise ValueError("empty conv1d output")
    cols = out_cols if out_cols is not None else (c * kernel + 63) // 64 * 64
    if out is None:
        out = torch.empty(b * lo, cols, dtype=torch.bfloat16, device=x.device)
    _check(out, "output", torch.bfloat16)
    if tuple(out.shape) != (b * lo, cols):
        raise ValueError(f"output must be {(b * lo, cols)}, got {tuple(out.shape)}")
    strides = (_lib.ctypes.c_int64 * 3)(x.stride(0), x.stride(2), x.stride(1))
    call("t2h_im2col_1d", ptr(x), _IN_DTYPES[x.dtype], strides, b, c, length, kernel, stride, padding, dilation, lo,
         ptr(out), cols, stream_handle())
    return out


def conv1d_q8_0(x: torch.Tensor, w: torch.Tensor, bias: torch.Tensor | None, kernel: int, *, stride: int = 1,
                padding: int = 0, dilation: int = 1, out_dtype: torch.dtype = torch.float32,
                residual: torch.Tensor | None = None) -> torch.Tensor:
    """CONV1D_Q8_0W_F32B_F32 on channels-last activations: x [B, L, C] -> [B, Lo, Co], W the reference's Q8_0
    rows [Co, C * K] (column c * K + k), bias fp32 [Co]; im2col_1d then the Q8_0 GEMM with the bias (and an fp32
    residual [B, Lo, Co]) in its epilogue."""
    b = int(x.shape[0])
    cols = im2col_1d(x, kernel, stride=stride, padding=padding, dilation=dilation)
    lo = cols.shape[0] // b
    out = torch.empty(b, lo, int(w.shape[0]), dtype=out_dtype, device=x.device)
    q8_0_linear(cols, w, bias=bias, out=out.view(b * lo, -1), out_dtype=out_dtype,
                residual=None if residual is None else residual.reshape(b * lo, -1))
    return out


def snake(x: torch.Tensor, alpha: torch.Tensor, *, eps: float = SNAKE_EPS, out: torch.Tensor | None = None) -> torch.Tensor:
    """x + sin(alpha x)^2 / (alpha + eps) per channel of channels-last fp32 x [..., C]; alpha fp32 [C]."""
    _check(x, "x", torch.float32)
    _check(alpha, "alpha", torch.float32)
    c = int(x.shape[-1])
    if alpha.numel() != c:
        raise ValueError(f"alpha must have {c} elements, got {alpha.numel()}")
    if out is None:
        out = torch.empty_like(x)
    _check(out, "output", torch.float32)
    if out.shape != x.shape:
        raise ValueError("output must have x's shape")
    call("t2h_snake", ptr(x), ptr(alpha), ptr(out), x.numel() // c, c, float(eps), stream_handle())
    return out


def conv_transpose1d_q8_0(x: torch.Tensor, w: torch.Tensor, bias: torch.Tensor | None, out_channels: int,
                          kernel: int, *, stride: int = 1, padding: int = 0, output_padding: int = 0) -> torch.Tensor:
    """CONV_TRANSPOSE1D_Q8_0W_F32B_F32 on channels-last fp32 x [B, L, Ci] -> [B, Lo, Co], Lo = (L - 1) stride -
    2 padding + kernel + output_padding (0 <= output_padding < stride); W the reference's Q8_0 rows
    [Ci, Co * kernel] as they are, bias fp32 [Co]."""
    if not isinstance(x, torch.Tensor) or x.device.type != "cuda" or x.dtype != torch.float32 or x.dim() != 3:
        raise ValueError("x must be fp32 [B, L, Ci] on a HIP device")
    _check(w, "weight", torch.uint8, align=2)
    b, length, ci = (int(d) for d in x.shape)
    blocks = (out_channels * kernel + 31) // 32
    if w.dim() != 2 or tuple(w.shape) != (ci, blocks * Q8_0_BYTES):
        raise ValueError(f"weight must be uint8 [{ci}, {blocks * Q8_0_BYTES}], got {tuple(w.shape)}")
    if bias is not None:
        _check(bias, "bias", torch.float32, align=4)
        if bias.numel() != out_channels:
            raise ValueError(f"bias must have {out_channels} elements")
    if not 0 <= output_padding < stride:
        raise ValueError(f"output_padding must be in [0, stride), got {output_padding}")
    lo = (length - 1) * stride - 2 * padding + kernel + output_padding
    if lo < 1:
        raise ValueError("empty output")
    out = torch.empty(b, lo, out_channels, dtype=torch.float32, device=x.device)
    strides = (_lib.ctypes.c_int64 * 3)(x.stride(0), x.stride(2), x.stride(1))
    call("t2h_conv_transpose1d_q8_0", ptr(x), strides, ptr(w), ptr(bias), ptr(out), b, ci, length, out_channels,
         kernel, stride, padding, lo, stream_handle())
    return out


def omnivoice_input_embed_q8_0(text_w: torch.Tensor, audio_w: torch.Tensor, ids: torch.Tensor,
                               audio_mask: torch.Tensor, vocab: int) -> torch.Tensor:
    """OMNIVOICE_INPUT_EMBED_Q8_0_F32: ids int64 [B, C, S], audio_mask uint32/int32 [B, S] -> fp32 [B, S, H]; text_w
    Q8_0 rows [n_text, H], audio_w Q8_0 rows [C * vocab, H]."""
    _check(text_w, "text_w", torch.uint8, align=2)
    _check(audio_w, "audio_w", torch.uint8, align=2)
    _check(ids, "ids", torch.int64, align=8)
    _check(audio_mask, "audio_mask", (torch.int32, torch.uint32), align=4)
    b, c, s = (int(d) for d in ids.shape)
    h = int(text_w.shape[1]) // Q8_0_BYTES * 32
    if int(audio_w.shape[1]) != int(text_w.shape[1]) or int(audio_w.shape[0]) != c * vocab:
        raise ValueError("audio_w must be Q8_0 rows [C * vocab, H] like text_w")
    if tuple(audio_mask.shape) != (b, s):
        raise ValueError(f"audio_mask must be [{b}, {s}]")
    out = torch.empty(b, s, h, dtype=torch.float32, device=ids.device)
    call("t2h_omnivoice_input_embed_q8_0", ptr(text_w), int(text_w.shape[0]), ptr(audio_w), ptr(ids), ptr(audio_mask),
         ptr(out), b, c, s, h, vocab, stream_handle())
    return out


def omnivoice_cfg_score(logits: torch.Tensor, tokens: torch.Tensor, *, codebooks: int, targets: int, vocab: int,
                        guidance: float, layer_penalty: float, temperature: float, step: int, seed: int,
                        mask_id: int) -> tuple[torch.Tensor, torch.Tensor]:
    """OMNIVOICE_CFG_SCORE_F32: fp32 logits [2, S, C * V], tokens int64 [C * T] -> (candidate tokens int64 [C * T],
    candidate scores fp32 [C * T])."""
    _check(logits, "logits", torch.float32)
    _check(tokens, "tokens", torch.int64, align=8)
    if logits.dim() != 3 or logits.shape[0] != 2 or logits.shape[2] != codebooks * vocab:
        raise ValueError(f"logits must be [2, S, {codebooks * vocab}], got {tuple(logits.shape)}")
    if tokens.numel() != codebooks * targets:
        raise ValueError("tokens must hold C * T values")
    ct = torch.empty(codebooks * targets, dtype=torch.int64, device=logits.device)
    cs = torch.empty(codebooks * targets, dtype=torch.float32, device=logits.device)
    call("t2h_omnivoice_cfg_score", ptr(logits), ptr(tokens), ptr(ct), ptr(cs), int(logits.shape[1]), codebooks,
         targets, vocab, float(guidance), float(layer_penalty), float(temperature), step & 0xffffffff,
         seed & 0xffffffff, int(mask_id), stream_handle())
    return ct, cs


def omnivoice_token_update_topk(cand_tokens: torch.Tensor, cand_scores: torch.Tensor, tokens: torch.Tensor,
                                batch_input_ids: torch.Tensor, *, unmask_count: int) -> None:
    """OMNIVOICE_TOKEN_UPDATE_TOPK_F32 in place on tokens int64 [C * T] and batch_input_ids int64 [2, C, S]."""
    for x, n, dt in ((cand_tokens, "cand_tokens", torch.int64), (cand_scores, "cand_scores", torch.float32),
                     (tokens, "tokens", torch.int64), (batch_input_ids, "batch_input_ids", torch.int64)):
        _check(x, n, dt, align=4)
    _, c, s = (int(d) for d in batch_input_ids.shape)
    n = tokens.numel()
    if n % c or cand_tokens.numel() != n or cand_scores.numel() != n:
        raise ValueError("candidates and tokens must hold C * T values")
    call("t2h_omnivoice_token_update_topk", ptr(cand_tokens), ptr(cand_scores), ptr(tokens), ptr(batch_input_ids), c,
         n // c, s, int(unmask_count), stream_handle())


# ----------------------------------------------- the reference's unfused operators --

def rope_table(cos: torch.Tensor, sin: torch.Tensor, start_position: int | torch.Tensor, *, theta: float,
               attention_scaling: float = 1.0) -> None:
    """cos / sin fp32 [B, T, D] of positions start_position + t (ROPE_TABLE_F32); ``start_position`` an int or a
    one-element int32 device tensor (read at run time, so a captured graph replays it)."""
    _check(cos, "cos", torch.float32, align=4)
    _check(sin, "sin", torch.float32, align=4)
    if cos.dim() != 3 or sin.shape != cos.shape:
        raise ValueError(f"cos and sin must be fp32 [B, T, D] of one shape, got {tuple(cos.shape)} {tuple(sin.shape)}")
    b, t_len, d = (int(x) for x in cos.shape)
    if isinstance(start_position, torch.Tensor):
        _check(start_position, "start_position", torch.int32, align=4)
        if start_position.numel() != 1:
            raise ValueError("start_position must have one element")
        start, start_ptr = 0, ptr(start_position)
    else:
        if int(start_position) < 0:
            raise ValueError("start_position must be non-negative")
        start, start_ptr = int(start_position), None
    call("t2h_rope_table", ptr(cos), ptr(sin), b, t_len, d, float(theta), start, start_ptr, float(attention_scaling),
         stream_handle())


def rms_norm_rope(x: torch.Tensor, weight: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, out: torch.Tensor, *,
                  transpose_out: bool, eps: float = RMS_EPS) -> torch.Tensor:
    """Per-head RMSNorm (D = 128) + RoPE from a table: x [B, T, G, D] fp32 / bf16, cos / sin fp32 [B, T, D] ->
    out [B, T, G, D], or [B, G, T, D] when ``transpose_out`` (RMS_NORM_ROPE_TRANSPOSE_F16,
    RMS_NORM_ROPE_TOKEN_F32)."""
    _check(x, "x", tuple(_OUT_DTYPES), align=4)
    _check(weight, "weight", torch.float32, align=4)
    _check(out, "output", tuple(_OUT_DTYPES), align=4)
    if x.dim() != 4:
        raise ValueError(f"x must be [B, T, G, D], got {tuple(x.shape)}")
    b, t_len, g, d = (int(v) for v in x.shape)
    for tab, name in ((cos, "cos"), (sin, "sin")):
        _check(tab, name, torch.float32, align=4)
        if tuple(tab.shape) != (b, t_len, d):
            raise ValueError(f"{name} must be [{b}, {t_len}, {d}], got {tuple(tab.shape)}")
    if weight.numel() != d:
        raise ValueError(f"weight must have {d} elements")
    want = (b, g, t_len, d) if transpose_out else (b, t_len, g, d)
    if tuple(out.shape) != want:
        raise ValueError(f"output must be {want}, got {tuple(out.shape)}")
    call("t2h_rms_norm_rope", ptr(x), _OUT_DTYPES[x.dtype], ptr(weight), ptr(cos), ptr(sin), ptr(out),
         _OUT_DTYPES[out.dtype], b, t_len, g, d, int(transpose_out), float(eps), stream_handle())
    return out


def kv_cache_write(src: torch.Tensor, positions: torch.Tensor, caches: list[torch.Tensor]) -> None:
    """src [B, T, H, D] (fp32 or bf16) into each bf16 cache [B, S_c, H, D] at positions int64 [T]
    (TOKEN_MAJOR_KV_CACHE_WRITE_F16_PAIR / _TRIPLE, TOKEN_MAJOR_VALUE_CACHE_WRITE_F32_TO_F16_PAIR / _TRIPLE)."""
    _check(src, "src", tuple(_OUT_DTYPES), align=4 if src.dtype == torch.bfloat16 else 8)
    _check(positions, "cache_position", torch.int64, align=8)
    if src.dim() != 4:
        raise ValueError(f"src must be [B, T, H, D], got {tuple(src.shape)}")
    b, t_len, h, d = (int(v) for v in src.shape)
    if positions.numel() != t_len:
        raise ValueError(f"cache_position must have {t_len} entries")
    if not 1 <= len(caches) <= 3:
        raise ValueError("one to three caches")
    for i, c in enumerate(caches):
        _check(c, f"cache_{i}", torch.bfloat16, align=4)
        if c.dim() != 4 or c.shape[0] != b or c.shape[2] != h or c.shape[3] != d:
            raise ValueError(f"cache_{i} must be bf16 [{b}, S, {h}, {d}], got {tuple(c.shape)}")
    arr = (ctypes.c_void_p * len(caches))(*[c.data_ptr() for c in caches])
    caps = (ctypes.c_uint32 * len(caches))(*[int(c.shape[1]) for c in caches])
    call("t2h_kv_cache_write", ptr(src), _OUT_DTYPES[src.dtype], ptr(positions), len(caches), ctypes.addressof(arr),
         ctypes.addressof(caps), b, t_len, h, d, stream_handle())


def token_select_chunks(scores: torch.Tensor, tokens: torch.Tensor, chunk_scores: torch.Tensor,
                        chunk_tokens: torch.Tensor) -> None:
    """The best (score, token) of each chunk of 1024 partials (QWEN3_TOKEN_SELECT_REDUCE_CHUNKS_F32)."""
    _check(scores, "scores", torch.float32, align=4)
    _check(tokens, "tokens", _TOKEN_DTYPES, align=4)
    _check(chunk_scores, "chunk_scores", torch.float32, align=4)
    _check(chunk_tokens, "chunk_tokens", _TOKEN_DTYPES, align=4)
    g = int(scores.numel())
    if tokens.numel() != g or g == 0:
        raise ValueError("scores and tokens must have the same non-zero length")
    c = -(-g // 1024)
    if chunk_scores.numel() != c or chunk_tokens.numel() != c:
        raise ValueError(f"{g} partials make {c} chunks")
    call("t2h_token_select_chunks", ptr(scores), ptr(tokens), g, ptr(chunk_scores), ptr(chunk_tokens),
         stream_handle())


def add(x: torch.Tensor, y: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """out = x + y elementwise, fp32 or bf16 (ADD_F32_PREFILL, ADD_F32_36); out may be x or y."""
    _check(x, "x", tuple(_OUT_DTYPES), align=2)
    _check(y, "y", x.dtype, align=2)
    if y.shape != x.shape:
        raise ValueError("x and y must have the same shape")
    if out is None:
        out = torch.empty_like(x)
    _check(out, "output", x.dtype, align=2)
    if out.shape != x.shape:
        raise ValueError("output must have the shape of x")
    call("t2h_add", ptr(x), ptr(y), ptr(out), _OUT_DTYPES[x.dtype], x.numel(), stream_handle())
    return out


def slice_last_token(x: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
    """out [B, 1, H] = x[:, -1] of fp32 x [B, S, H] (SLICE_LAST_TOKEN_F32_TO_F16)."""
    _check(x, "x", torch.float32, align=4)
    _check(out, "output", tuple(_OUT_DTYPES), align=2)
    if x.dim() != 3:
        raise ValueError(f"x must be [B, S, H], got {tuple(x.shape)}")
    b, s_len, h = (int(v) for v in x.shape)
    if tuple(out.shape) != (b, 1, h):
        raise ValueError(f"output must be [{b}, 1, {h}], got {tuple(out.shape)}")
    call("t2h_slice_last_token", ptr(x), ptr(out), _OUT_DTYPES[out.dtype], b, s_len, h, stream_handle())
    return out
