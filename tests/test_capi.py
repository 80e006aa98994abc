"""The C ABI library on the CPU: it loads, exports every declared symbol, and rejects bad arguments
before any launch (no GPU is touched: every call here returns from host-side validation)."""

from __future__ import annotations

import ctypes
import subprocess

import pytest

from torch2vk_amd import _lib


@pytest.fixture(scope="module")
def lib():
    if not _lib.LIB_PATH.exists():
        pytest.skip("libt2h.so not built")
    return _lib.lib()


def test_exports_every_declared_symbol(lib):
    declared = _lib.declared_symbols()
    assert len(declared) >= 15
    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)], capture_output=True, text=True,
                         check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if line.strip()}
    missing = [s for s in declared if s not in exported]
    assert not missing, f"declared in include/t2h.h but not exported: {missing}"
    # and the Python binding covers every entry point
    assert set(declared) <= set(_lib.SIGNATURES), set(declared) - set(_lib.SIGNATURES)


def test_status_strings(lib):
    assert lib.t2h_abi_version() == 1
    assert lib.t2h_status_string(0) == b"ok"
    assert b"null" in lib.t2h_status_string(1)
    assert lib.t2h_status_string(1000 + 1) == b"HIP launch error"


def test_argument_validation_returns_status(lib):
    fake = ctypes.c_void_p(0x1000)  # never dereferenced: validation fails first
    # null pointers
    assert lib.t2h_q4k_matvec(None, fake, fake, 0, None, 1, 4096, 16, None) == 1
    assert lib.t2h_quantize_q4_k(None, 4, 256, fake, None) == 1
    # K not a multiple of 256
    assert lib.t2h_q4k_matvec(fake, fake, fake, 0, None, 1, 1000, 16, None) == 2
    assert lib.t2h_quantize_q4_k(fake, 4, 300, fake, None) == 2
    assert lib.t2h_quantize_q8_0(fake, 4, 33, fake, None) == 2
    # K a multiple of 256 but not built (NSB 5)
    assert lib.t2h_q4k_matvec(fake, fake, fake, 0, None, 1, 1280, 16, None) == 4
    # N not a multiple of the row group (K=256 -> 16 rows per group)
    assert lib.t2h_q4k_matvec(fake, fake, fake, 0, None, 1, 256, 10, None) == 2
    # bad dtype combination: bf16 output with a residual
    assert lib.t2h_q4k_matvec(fake, fake, fake, 1, fake, 1, 4096, 16, None) == 3
    # attention: head_dim other than 128, GQA not dividing, too-small workspace
    assert lib.t2h_attn_decode(fake, fake, fake, None, None, 1e-6, 0.0, fake, fake, fake, 32, 8, 64, 64, fake, fake,
                               1 << 20, None) == 4
    assert lib.t2h_attn_decode(fake, fake, fake, None, None, 1e-6, 0.0, fake, fake, fake, 30, 8, 128, 64, fake, fake,
                               1 << 20, None) == 2
    assert lib.t2h_attn_decode(fake, fake, fake, None, None, 1e-6, 0.0, fake, fake, fake, 32, 8, 128, 4096, fake, fake,
                               16, None) == 6
    # workspace sizing is pure host arithmetic
    assert lib.t2h_attn_decode_workspace_bytes(32, 8, 128, 4352) > 0
    assert lib.t2h_attn_decode_workspace_bytes(32, 8, 64, 4352) == 0
    assert lib.t2h_set_gemv_max_blocks(0, 0) == 5
    # Q6_K / Q8_0 GEMV: K rule, rows too long or too short for the built geometries, row-group multiple
    assert lib.t2h_q6k_matvec(fake, fake, fake, 0, None, 1, 1000, 16, None) == 2
    assert lib.t2h_q6k_matvec(fake, fake, fake, 0, None, 1, 16384, 16, None) == 4
    assert lib.t2h_q6k_matvec(fake, fake, fake, 0, None, 1, 256, 16, None) == 4
    assert lib.t2h_q6k_matvec(fake, fake, fake, 0, None, 1, 1024, 6, None) == 2   # 4 rows per group at K=1024
    assert lib.t2h_q8_0_matvec(fake, fake, fake, 0, None, 1, 48, 16, None) == 2
    assert lib.t2h_q8_0_matvec(fake, fake, fake, 0, None, 1, 256, 16, None) == 4
    assert lib.t2h_q8_0_matvec(None, fake, fake, 0, None, 1, 1024, 16, None) == 1
    assert lib.t2h_q6k_rmsnorm_matvec(fake, None, 1e-6, fake, fake, 0, 1024, 16, None) == 1
    assert lib.t2h_q6k_lm_head_argmax_partial(fake, None, 1e-6, fake, 4096, 100, fake, fake, 0, None) == 5
    # the LM head of several sequences: sequence count, built k, row multiple, partial count, null arrays
    arr = (ctypes.c_void_p * 4)(fake, fake, fake, fake)
    pa = ctypes.addressof(arr)
    assert lib.t2h_q4k_lm_head_argmax_partial_seqs(0, pa, fake, 1e-6, fake, 1024, 64, pa, pa, 8, None) == 5
    assert lib.t2h_q4k_lm_head_argmax_partial_seqs(5, pa, fake, 1e-6, fake, 1024, 64, pa, pa, 8, None) == 5
    assert lib.t2h_q4k_lm_head_argmax_partial_seqs(2, pa, fake, 1e-6, fake, 2048, 64, pa, pa, 8, None) == 4
    assert lib.t2h_q4k_lm_head_argmax_partial_seqs(2, pa, fake, 1e-6, fake, 1024, 66, pa, pa, 8, None) == 2
    assert lib.t2h_q4k_lm_head_argmax_partial_seqs(2, pa, fake, 1e-6, fake, 1024, 64, pa, pa, 0, None) == 5
    assert lib.t2h_q4k_lm_head_argmax_partial_seqs(2, None, fake, 1e-6, fake, 1024, 64, pa, pa, 8, None) == 1
    assert lib.t2h_embedding_q4_k_seqs(0, fake, 10, pa, 1024, pa, None) == 5
    assert lib.t2h_embedding_q4_k_seqs(2, fake, 10, pa, 1000, pa, None) == 2
    assert lib.t2h_embedding_q4_k_seqs(2, None, 10, pa, 1024, pa, None) == 1
    # weights read with 16-byte loads: a misaligned weight pointer is refused
    odd = ctypes.c_void_p(0x1001)
    assert lib.t2h_q4k_lm_head_argmax_partial_seqs(2, pa, fake, 1e-6, odd, 1024, 64, pa, pa, 8, None) == 7
    assert lib.t2h_embedding_q4_k_seqs(2, odd, 10, pa, 1024, pa, None) == 7
    assert lib.t2h_embedding_q4_k(odd, 10, fake, 1, 1024, fake, None) == 7
    assert lib.t2h_embedding_q4_k(fake, 10, fake, 1, 1024, odd, None) == 7
    # the unfused operators: null pointers, dtype codes, head_dim, cache count, alignment
    assert lib.t2h_rope_table(None, fake, 1, 4, 128, 1e6, 0, None, 1.0, None) == 1
    assert lib.t2h_rope_table(fake, fake, 1, 4, 127, 1e6, 0, None, 1.0, None) == 2
    assert lib.t2h_rope_table(fake, fake, 1, 4, 128, 0.0, 0, None, 1.0, None) == 2
    assert lib.t2h_rms_norm_rope(fake, 0, fake, fake, fake, fake, 0, 1, 4, 2, 64, 0, 1e-6, None) == 4
    assert lib.t2h_rms_norm_rope(fake, 7, fake, fake, fake, fake, 0, 1, 4, 2, 128, 0, 1e-6, None) == 3
    assert lib.t2h_rms_norm_rope(fake, 0, None, fake, fake, fake, 0, 1, 4, 2, 128, 0, 1e-6, None) == 1
    caps = (ctypes.c_uint32 * 4)(8, 8, 8, 8)
    cp = ctypes.addressof(caps)
    assert lib.t2h_kv_cache_write(fake, 1, fake, 0, pa, cp, 1, 2, 2, 128, None) == 5
    assert lib.t2h_kv_cache_write(fake, 1, fake, 4, pa, cp, 1, 2, 2, 128, None) == 5
    assert lib.t2h_kv_cache_write(ctypes.c_void_p(0x1002), 1, fake, 2, pa, cp, 1, 2, 2, 128, None) == 7
    assert lib.t2h_kv_cache_write(fake, 2, fake, 2, pa, cp, 1, 2, 2, 128, None) == 3
    assert lib.t2h_token_select_chunks(fake, fake, 0, fake, fake, None) == 2
    assert lib.t2h_token_select_chunks(None, fake, 8, fake, fake, None) == 1
    assert lib.t2h_add(fake, fake, fake, 5, 16, None) == 3
    assert lib.t2h_slice_last_token(fake, fake, 0, 1, 0, 16, None) == 2
    assert lib.t2h_token_select_store_seqs(5, pa, pa, 8, fake, 1, pa, pa, pa, 4, pa, pa, 1, pa, None) == 5
    assert lib.t2h_token_select_store_seqs(2, pa, pa, 0, fake, 1, pa, pa, pa, 4, pa, pa, 1, pa, None) == 2
    assert lib.t2h_token_select_store_seqs(2, pa, pa, 8, None, 1, pa, pa, pa, 4, pa, pa, 1, pa, None) == 1
    # bf16-weight GEMM and the dequantise-once kernel: nulls, K rule, 16-byte operands, weight type codes
    assert lib.t2h_bf16_gemm(None, fake, fake, 0, None, 4, 128, 16, None) == 1
    assert lib.t2h_bf16_gemm(fake, fake, fake, 0, None, 4, 100, 16, None) == 2
    assert lib.t2h_bf16_gemm(odd, fake, fake, 0, None, 4, 128, 16, None) == 7
    assert lib.t2h_bf16_gemm(fake, odd, fake, 0, None, 4, 128, 16, None) == 7
    assert lib.t2h_bf16_gemm(fake, fake, fake, 9, None, 4, 128, 16, None) == 3
    assert lib.t2h_dequantize_bf16(99, fake, 4, 256, fake, None) == 3
    assert lib.t2h_dequantize_bf16(8, None, 4, 256, fake, None) == 1
    assert lib.t2h_dequantize_bf16(12, fake, 4, 320, fake, None) == 2   # Q4_K: K % 256
    assert lib.t2h_dequantize_bf16(8, fake, 4, 96, fake, None) == 2     # K % 64
    assert lib.t2h_dequantize_bf16(8, fake, 4, 256, odd, None) == 7
    assert lib.t2h_gemm_swiglu(30, fake, fake, fake, fake, 4, 100, 16, None) == 2
    assert lib.t2h_gemm_swiglu(30, fake, odd, fake, fake, 4, 128, 16, None) == 7
    # the traced multi-sequence decode launch checks its timeline buffer before anything else
    assert lib.t2h_qwen3_decode_layers_seqs_traced(4, pa, 28, 1024, 3072, 16, 8, 128, 512, pa, pa, 1e-6, 1e6, pa,
                                                   1 << 20, pa, None, 1 << 20, None) == 1
    assert lib.t2h_qwen3_decode_layers_seqs_traced(4, pa, 28, 1024, 3072, 16, 8, 128, 512, pa, pa, 1e-6, 1e6, pa,
                                                   1 << 20, pa, fake, 64, None) == 6
    assert lib.t2h_qwen3_decode_layers_seqs_traced(4, pa, 28, 1024, 3072, 16, 8, 128, 512, pa, pa, 1e-6, 1e6, pa,
                                                   1 << 20, pa, ctypes.c_void_p(0x1004), 1 << 24, None) == 7


def test_python_wrappers_reject_host_tensors():
    import torch

    from torch2vk_amd import kernels

    with pytest.raises(ValueError, match="HIP device"):
        kernels.quantize(torch.zeros(4, 256), "q4_k")
    with pytest.raises(ValueError, match="HIP device"):
        kernels.q4k_matvec(torch.zeros(256, dtype=torch.bfloat16), torch.zeros(16, 144, dtype=torch.uint8))


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(_lib, "LIB_PATH", tmp_path / "libt2h.so")
    monkeypatch.setattr(_lib, "_lib", None)
    with pytest.raises(RuntimeError, match="missing"):
        _lib.lib()
