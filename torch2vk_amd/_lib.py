"""ctypes binding of libt2h.so (the C ABI declared in include/t2h.h).

torch is imported first so that libt2h resolves ``libamdhip64.so.7`` to the
HIP runtime torch already loaded: one runtime, shared streams.  There is no
fallback: if the library is missing, every call raises.
"""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import torch  # noqa: F401  (must precede loading libt2h, see module docstring)

PKG = Path(__file__).resolve().parent
LIB_PATH = PKG / "libt2h.so"
HEADER = PKG.parent / "include" / "t2h.h"

T2H_OK = 0
T2H_DTYPE_F32 = 0
T2H_DTYPE_BF16 = 1
T2H_WTYPE_Q4_K = 12
T2H_WTYPE_Q6_K = 14
T2H_WTYPE_Q8_0 = 8
T2H_WTYPE_BF16 = 30

_vp = ctypes.c_void_p
_u32 = ctypes.c_uint32
_u64 = ctypes.c_uint64
_i32 = ctypes.c_int
_f32 = ctypes.c_float
_sz = ctypes.c_size_t

# name -> (restype, argtypes)
SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "t2h_abi_version": (_i32, []),
    "t2h_status_string": (ctypes.c_char_p, [_i32]),
    "t2h_quantize_q4_k": (_i32, [_vp, _u32, _u32, _vp, _vp]),
    "t2h_quantize_q6_k": (_i32, [_vp, _u32, _u32, _vp, _vp]),
    "t2h_quantize_q8_0": (_i32, [_vp, _u32, _u32, _vp, _vp]),
    "t2h_dequantize": (_i32, [_i32, _vp, _u32, _u32, _vp, _vp]),
    "t2h_q4k_matvec": (_i32, [_vp, _vp, _vp, _i32, _vp, _u32, _u32, _u32, _vp]),
    "t2h_q4k_matvec_multi": (_i32, [_vp, _vp, _f32, _u32, _vp, _vp, _vp, _u32, _i32, _vp]),
    "t2h_q4k_rmsnorm_swiglu_matvec": (_i32, [_vp, _vp, _f32, _vp, _vp, _vp, _u32, _u32, _vp]),
    "t2h_q4k_lm_head_argmax_partial": (_i32, [_vp, _vp, _f32, _vp, _u32, _u32, _vp, _vp, _u32, _vp]),
    "t2h_q4k_lm_head_argmax_partial_seqs": (_i32, [_u32, _vp, _vp, _f32, _vp, _u32, _u32, _vp, _vp, _u32,
                                                    _vp]),
    "t2h_set_gemv_max_blocks": (_i32, [_u32, _u32]),
    "t2h_q6k_matvec": (_i32, [_vp, _vp, _vp, _i32, _vp, _u32, _u32, _u32, _vp]),
    "t2h_q6k_rmsnorm_matvec": (_i32, [_vp, _vp, _f32, _vp, _vp, _i32, _u32, _u32, _vp]),
    "t2h_q8_0_matvec": (_i32, [_vp, _vp, _vp, _i32, _vp, _u32, _u32, _u32, _vp]),
    "t2h_matvec_supported": (_i32, [_i32, _u32, _u32]),
    "t2h_q8_0_gemm": (_i32, [_vp, _vp, _vp, _i32, _vp, _u32, _u32, _u32, _vp]),
    "t2h_q4k_gemm": (_i32, [_vp, _vp, _vp, _i32, _vp, _u32, _u32, _u32, _vp]),
    "t2h_q6k_lm_head_argmax_partial": (_i32, [_vp, _vp, _f32, _vp, _u32, _u32, _vp, _vp, _u32, _vp]),
    "t2h_token_select": (_i32, [_vp, _vp, _u32, _vp, _u32, _vp, _vp, _vp]),
    "t2h_token_store": (_i32, [_vp, _vp, _vp, _u32, _vp, _vp, _u32, _vp, _u32, _vp, _vp]),
    "t2h_token_select_store": (_i32, [_vp, _vp, _u32, _vp, _u32, _vp, _vp, _vp, _u32, _vp, _vp, _u32, _vp, _vp]),
    "t2h_token_select_store_seqs": (_i32, [_u32, _vp, _vp, _u32, _vp, _u32, _vp, _vp, _vp, _u32, _vp, _vp, _u32,
                                            _vp, _vp]),
    "t2h_attn_decode_workspace_bytes": (_sz, [_u32, _u32, _u32, _u32]),
    "t2h_attn_decode": (_i32, [_vp, _vp, _vp, _vp, _vp, _f32, _f32, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _vp,
                              _vp, _sz, _vp]),
    "t2h_qwen3_decode_layers_workspace_bytes": (_sz, [_u32, _u32, _u32, _u32, _u32]),
    "t2h_qwen3_decode_layers": (_i32, [_vp, _u32, _u32, _u32, _u32, _u32, _u32, _u32, _vp, _vp, _f32, _f32, _vp,
                                       _sz, _vp, _vp]),
    "t2h_qwen3_decode_layers_noalloc": (_i32, [_vp, _u32, _u32, _u32, _u32, _u32, _u32, _u32, _vp, _vp, _f32, _f32,
                                               _vp, _vp]),
    "t2h_qwen3_decode_layers_seqs": (_i32, [_u32, _vp, _u32, _u32, _u32, _u32, _u32, _u32, _u32, _vp, _vp, _f32,
                                             _f32, _vp, _sz, _vp, _vp]),
    "t2h_qwen3_decode_layers_trace_bytes": (_sz, [_u32]),
    "t2h_qwen3_decode_layers_seqs_traced": (_i32, [_u32, _vp, _u32, _u32, _u32, _u32, _u32, _u32, _u32, _vp, _vp,
                                                   _f32, _f32, _vp, _sz, _vp, _vp, _sz, _vp]),
    "t2h_qwen3_decode_layers_traced": (_i32, [_vp, _u32, _u32, _u32, _u32, _u32, _u32, _u32, _vp, _vp, _f32, _f32,
                                              _vp, _sz, _vp, _vp, _sz, _vp]),
    "t2h_flash_attn_prefill": (_i32, [_vp, _vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _u32, _u32, _vp, _i32,
                                      ctypes.c_int32, _f32, _vp]),
    "t2h_flash_attn_prefill_tiles": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _u32, _u32, _vp,
                                            _i32, ctypes.c_int32, _f32, _vp]),
    "t2h_fa_mask_tiles": (_i32, [_vp, _u32, _u32, _u32, ctypes.c_int64, ctypes.c_int64, _vp, _vp]),
    "t2h_embedding_q4_k": (_i32, [_vp, _u64, _vp, _u32, _u32, _vp, _vp]),
    "t2h_embedding_q4_k_seqs": (_i32, [_u32, _vp, _u64, _vp, _u32, _vp, _vp]),
    "t2h_rms_norm": (_i32, [_vp, _i32, _vp, _vp, _i32, _u32, _u32, _f32, _vp]),
    "t2h_swiglu": (_i32, [_vp, _vp, _i32, _vp, _u64, _vp]),
    "t2h_q8_0_linear": (_i32, [_vp, _vp, _vp, _i32, _vp, _i32, _vp, _u32, _u32, _u32, _u32, _vp]),
    "t2h_flash_attn_segments": (_i32, [_vp, _vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _u32, _u32, _vp, _f32,
                                       _vp]),
    "t2h_im2col": (_i32, [_vp, _i32, _vp, _u32, _u32, _u32, _u32, _u32, _u32, _u32, _u32, _u32, _u32, _u32, _u32,
                          _vp, _u32, _vp]),
    "t2h_layer_norm": (_i32, [_vp, _i32, _vp, _vp, _vp, _i32, _u32, _u32, _f32, _vp]),
    "t2h_gelu": (_i32, [_vp, _i32, _vp, _i32, _u64, _vp]),
    "t2h_index_select_rows": (_i32, [_vp, _u64, _u32, _vp, _u32, _vp, _vp]),
    "t2h_index_copy_rows": (_i32, [_vp, _u64, _u32, _vp, _u32, _vp, _vp]),
    "t2h_embedding_q8_0": (_i32, [_vp, _u64, _vp, _u32, _u32, _vp, _vp]),
    "t2h_q6k_gemm": (_i32, [_vp, _vp, _vp, _i32, _vp, _u32, _u32, _u32, _vp]),
    "t2h_bf16_gemm": (_i32, [_vp, _vp, _vp, _i32, _vp, _u32, _u32, _u32, _vp]),
    "t2h_bf16_linear": (_i32, [_vp, _vp, _vp, _i32, _vp, _i32, _vp, _u32, _u32, _u32, _vp]),
    "t2h_dequantize_bf16": (_i32, [_i32, _vp, _u32, _u32, _vp, _vp]),
    "t2h_gemm_swiglu": (_i32, [_i32, _vp, _vp, _vp, _vp, _u32, _u32, _u32, _vp]),
    "t2h_gemm_splitk_bytes": (_sz, [_u32, _u32, _u32, _i32]),
    "t2h_gemm_splitk": (_i32, [_i32, _vp, _vp, _vp, _vp, _i32, _vp, _i32, _vp, _u32, _u32, _u32, _u32, _u32, _vp, _sz,
                               _vp]),
    "t2h_im2col_1d": (_i32, [_vp, _i32, _vp, _u32, _u32, _u32, _u32, _u32, _u32, _u32, _u32, _vp, _u32, _vp]),
    "t2h_snake": (_i32, [_vp, _vp, _vp, _u64, _u32, _f32, _vp]),
    "t2h_conv_transpose1d_q8_0": (_i32, [_vp, _vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _u32, _u32, _u32, _u32,
                                         _vp]),
    "t2h_omnivoice_input_embed_q8_0": (_i32, [_vp, _u32, _vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _u32, _vp]),
    "t2h_omnivoice_cfg_score": (_i32, [_vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _f32, _f32, _f32, _u32, _u32,
                                       ctypes.c_int64, _vp]),
    "t2h_omnivoice_token_update_topk": (_i32, [_vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _vp]),
    "t2h_qk_norm_rope_cache": (_i32, [_vp, _u64, _vp, _u64, _vp, _u64, _vp, _vp, _f32, _f32, ctypes.c_int32, _u32,
                                      _u32, _u32, _u32, _vp, _vp, _vp, _u32, _vp]),
    "t2h_qk_norm_rope_cache_seqs": (_i32, [_vp, _u64, _vp, _u64, _vp, _u64, _vp, _vp, _f32, _f32, ctypes.c_int32,
                                           _u32, _u32, _u32, _u32, _u32, _vp, _vp, _vp, _u32, _vp]),
    "t2h_rope_table": (_i32, [_vp, _vp, _u32, _u32, _u32, _f32, _u32, _vp, _f32, _vp]),
    "t2h_rms_norm_rope": (_i32, [_vp, _i32, _vp, _vp, _vp, _vp, _i32, _u32, _u32, _u32, _u32, _i32, _f32, _vp]),
    "t2h_kv_cache_write": (_i32, [_vp, _i32, _vp, _u32, _vp, _vp, _u32, _u32, _u32, _u32, _vp]),
    "t2h_token_select_chunks": (_i32, [_vp, _vp, _u32, _vp, _vp, _vp]),
    "t2h_add": (_i32, [_vp, _vp, _vp, _i32, _u64, _vp]),
    "t2h_slice_last_token": (_i32, [_vp, _vp, _i32, _u32, _u32, _u32, _vp]),
}


class T2HError(RuntimeError):
    """A libt2h entry point returned a non-zero status."""

    def __init__(self, fn: str, status: int, detail: str) -> None:
        super().__init__(f"{fn} failed with status {status}: {detail}")
        self.status = status


_lib: ctypes.CDLL | None = None


def declared_symbols() -> list[str]:
    """Every function name declared in include/t2h.h."""
    text = HEADER.read_text()
    return sorted(set(re.findall(r"\b(t2h_[a-z0-9_]+)\s*\(", text)))


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build the HIP library first (python -m torch2vk_amd.build)")
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = handle
    return _lib


def call(name: str, *args) -> None:
    """Call a status-returning entry point and raise T2HError on failure."""
    status = getattr(lib(), name)(*args)
    if status != T2H_OK:
        detail = lib().t2h_status_string(status).decode()
        raise T2HError(name, status, detail)


def stream_handle(stream: torch.cuda.Stream | None = None) -> int:
    s = stream if stream is not None else torch.cuda.current_stream()
    return int(s.cuda_stream)


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else int(t.data_ptr())
