"""The reference-named operator surface on the host: contract checks and symbol binding raise before any launch
(the reference's dispatcher errors, src/torch2vk/runtime/dispatcher.py:28-53), weight layouts are recognised
from the reference's physical types, and the variant names match the reference shaders'."""

from __future__ import annotations

import pytest
import torch

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
    add,
    ceil_div,
    eval_expr,
    mul,
    weight_layout,
)


def _probe_variant(log):
    fields = (TensorFieldSpec("x", IOKind.INPUT, "input", TensorContract("bfloat16", ("X0", "X1", "K"))),
              TensorFieldSpec("weight", IOKind.INPUT, "weight",
                              TensorContract("uint32", ("N", mul(ceil_div("K", 256), 36)), Q4_K_WORDS)),
              TensorFieldSpec("output", IOKind.OUTPUT, "output", TensorContract(("float32", "bfloat16"),
                                                                              ("X0", "X1", "N"))))
    contract = ShaderContract("Probe", "probe", fields, (PushConstantInput("cache_position"),))
    return ShaderVariant("probe", "test", contract, lambda rt, t, sym, push: log.append((dict(sym), dict(push))))


def _args(m=1, k=512, n=64):
    return dict(x=torch.zeros(1, m, k, dtype=torch.bfloat16), weight=torch.zeros(n, k // 256 * 36, dtype=torch.uint32),
                output=torch.zeros(1, m, n), cache_position=7)


def test_eval_expr_matches_the_reference_semantics():
    sym = {"K": 1000, "N": 3}
    assert eval_expr(mul(ceil_div("K", 256), 36), sym) == 4 * 36
    assert eval_expr(add("N", 2), sym) == 5 and eval_expr(17, sym) == 17
    with pytest.raises(ValueError, match="Unresolved shape symbol"):
        eval_expr("M", sym)
    with pytest.raises(ValueError, match="rhs must be positive"):
        eval_expr(ceil_div("K", 0), sym)


def test_dispatch_binds_symbols_and_launches_once():
    log = []
    rt = RuntimeSession("cpu")
    _probe_variant(log)(rt, **_args(m=3))
    assert log == [({"X0": 1, "X1": 3, "K": 512, "N": 64}, {"cache_position": 7})]


@pytest.mark.parametrize("mutate,exc,match", [
    (lambda a: a.pop("output"), ValueError, "missing tensor fields"),
    (lambda a: a.pop("cache_position"), ValueError, "missing push constant inputs"),
    (lambda a: a.update(bias=torch.zeros(1)), ValueError, "unexpected fields"),
    (lambda a: a.update(x=[1, 2]), TypeError, "expects a tensor"),
    (lambda a: a.update(x=torch.zeros(1, 1, 512)), TypeError, "dtype"),
    (lambda a: a.update(weight=torch.zeros(64, 36, dtype=torch.uint32)), ValueError, "axis 1"),
    (lambda a: a.update(output=torch.zeros(1, 1, 65)), ValueError, "axis 2"),
    (lambda a: a.update(x=torch.zeros(1, 512, dtype=torch.bfloat16)), ValueError, "rank"),
    (lambda a: a.update(output=torch.zeros(1, 1, 128)[:, :, ::2]), ValueError, "contiguous"),
    (lambda a: a.update(cache_position=-1), TypeError, "non-negative"),
    (lambda a: a.update(cache_position=torch.zeros(2, dtype=torch.int32)), TypeError, "one-element"),
])
def test_dispatch_rejects_before_launch(mutate, exc, match):
    log = []
    args = _args()
    mutate(args)
    with pytest.raises(exc, match=match):
        _probe_variant(log)(RuntimeSession("cpu"), **args)
    assert log == []


def test_weight_layout_from_physical_type():
    k = 1024
    assert weight_layout(torch.zeros(8, k // 256 * 36, dtype=torch.uint32), k) == Q4_K_WORDS
    assert weight_layout(torch.zeros(8, k // 256 * 105, dtype=torch.uint16), k) == Q6_K_HALFWORDS
    assert weight_layout(torch.zeros(8, k // 32 * 17, dtype=torch.uint16), k) == Q8_0_HALFWORDS
    assert weight_layout(torch.zeros(8, 40 // 32 * 17 + 17, dtype=torch.uint16), 40) == Q8_0_HALFWORDS  # K % 32 != 0
    with pytest.raises(ValueError, match="expected Q4_K, Q6_K, or Q8_0"):
        weight_layout(torch.zeros(8, 100, dtype=torch.uint8), k)


def test_reference_variant_names():
    from torch2vk_amd import variants as V

    names = {v.name for v in vars(V).values() if isinstance(v, ShaderVariant)}
    for n in ("linear_nobias_q4_k_matvec_f32", "linear_nobias_q4_k_matvec_add_f32", "linear_nobias_q6_k_matvec_f32",
              "linear_nobias_q6_k_matvec_add_f32", "linear_nobias_q8_0_matvec_f32", "linear_nobias_q4_k_qkv_matvec_f32",
              "linear_nobias_q4_k_qk_matvec_f32", "linear_nobias_q4_qk_q6_v_matvec_f32", "linear_nobias_q4_k_f32",
              "linear_nobias_q8_0_f32", "rms_norm_mul_f16_f32", "swiglu_f16", "embedding_q4_k_f32",
              "sdpa_decode_cache_write_f32",
              # the rest of the decode step and the prefill (src/models/optimized_qwen3/dispatch/*.py, run.py)
              "lm_head_q6_k_argmax_partial_f16", "qwen3_token_select_reduce_chunks_f32",
              "qwen3_token_select_reduce_f32", "qwen3_token_store_eos_f32", "qwen3_token_store_eos",
              "qwen3_token_store", "rms_norm_rope_transpose_f16", "rope_table_f32", "rms_norm_rope_token_f32",
              "rms_norm_rope_token_f32_to_f16", "llama_flash_attn_f32_f16_f16", "fa_mask_opt_f16",
              "llama_matmul_q4_k_f32_m", "llama_matmul_q4_k_f32_l", "llama_matmul_q6_k_f32_m",
              "llama_matmul_q6_k_f32_l", "embedding_q4_k_act_f32", "embedding_q8_0_f32", "rms_norm_mul_f32",
              "add_f32_prefill", "add_f32_36", "slice_last_token_f32_to_f16", "swiglu_f32",
              "token_major_kv_cache_write_f16_pair", "token_major_kv_cache_write_f16_triple",
              "token_major_value_cache_write_f32_to_f16_pair", "token_major_value_cache_write_f32_to_f16_triple"):
        assert n in names, n
    # the variant the rows select, as make_linear_nobias_q4_k_m_variant does
    assert V.linear_nobias_quantized_variant(1, Q4_K_WORDS) is V.LINEAR_NOBIAS_Q4_K_MATVEC_F32
    assert V.linear_nobias_quantized_variant(8, Q8_0_HALFWORDS) is V.LINEAR_NOBIAS_Q8_0_MATVEC_F32
    assert V.linear_nobias_quantized_variant(9, Q4_K_WORDS) is V.LINEAR_NOBIAS_Q4_K_F32
    assert V.linear_nobias_quantized_variant(9, Q6_K_HALFWORDS) is V.LINEAR_NOBIAS_Q6_K_F32


def test_matvec_variant_refuses_more_than_eight_rows():
    from torch2vk_amd import variants as V

    rt = RuntimeSession("cpu")
    args = dict(x=torch.zeros(1, 9, 256, dtype=torch.bfloat16), weight=torch.zeros(16, 36, dtype=torch.uint32),
                output=torch.zeros(1, 9, 16))
    with pytest.raises(ValueError, match="at most 8 rows"):
        V.LINEAR_NOBIAS_Q4_K_MATVEC_F32(rt, **args)


def test_run_decode_layer_needs_bound_tensors():
    import torch2vk_amd.qwen3.dispatch as D

    D._MODEL = None
    with pytest.raises(RuntimeError, match="bind_model_tensors"):
        D.run_decode_layer(RuntimeSession("cpu"), 0, cache_position=0)


def test_matvec_shape_query():
    """The GEMV shape query the linear dispatcher consults (host-only, no device work)."""
    from torch2vk_amd import kernels

    assert kernels.matvec_supported("q4_k", 4096, 12288) and kernels.matvec_supported("q4_k", 12288, 4096)
    assert kernels.matvec_supported("q4_k", 1024, 2048)
    assert not kernels.matvec_supported("q4_k", 2560, 64)       # 10 superblocks per row: not built
    assert kernels.matvec_supported("q6_k", 1024, 80) and kernels.matvec_supported("q6_k", 12288, 4096)
    assert not kernels.matvec_supported("q6_k", 512, 80)        # 8 rows per unit: not built
    assert not kernels.matvec_supported("q6_k", 1024, 82)       # N not a multiple of the 4 rows per unit
    assert not kernels.matvec_supported("q6_k", 16384, 64)      # longer rows than the register-resident x
    assert kernels.matvec_supported("q8_0", 512, 80) and not kernels.matvec_supported("q8_0", 256, 8)
    assert not kernels.matvec_supported("q4_k", 1000, 64)       # not a whole number of superblocks


def test_named_dispatch_functions_exist_and_need_bound_tensors():
    """The reference's dispatch function names (src/models/optimized_qwen3/dispatch/*.py) are all here, and each
    refuses to run before bind_model_tensors / bind_prefill_tensors."""
    import torch2vk_amd.qwen3.dispatch as D

    for name in ("run_decode_embed", "run_decode_layer", "run_decode_norm", "run_prefill_full_embed",
                 "run_prefill_tail_embed", "run_prefill_full_layer", "run_prefill_tail_layer",
                 "run_prefill_tail_last_layer_tail", "run_prefill_full_mask_opt", "run_prefill_tail_mask_opt",
                 "run_text_norm", "run_lm_head_select", "run_token_store", "run_decode_step", "run_prefill"):
        assert callable(getattr(D, name)), name
    D._MODEL = None
    rt = RuntimeSession("cpu")
    with pytest.raises(RuntimeError, match="bind_model_tensors"):
        D.run_decode_embed(rt)
    with pytest.raises(RuntimeError, match="bind_model_tensors"):
        D.run_prefill_tail_layer(rt, 0)


def test_float_push_input():
    """ROPE_TABLE_F32's theta is a float push input: a number is taken, a tensor or a string is refused before
    the launch; start_position stays an unsigned input."""
    from torch2vk_amd import variants as V

    log = []
    probe = ShaderVariant("probe_rope", "test", ShaderContract(
        "Probe", "probe_rope", V.ROPE_TABLE_F32.contract.fields, V.ROPE_TABLE_F32.contract.push_inputs),
        lambda rt, t, sym, push: log.append(dict(push)))
    rt = RuntimeSession("cpu")
    cos, sin = torch.zeros(1, 3, 128), torch.zeros(1, 3, 128)
    probe(rt, cos=cos, sin=sin, theta=1e6, start_position=7)
    assert log == [{"theta": 1e6, "start_position": 7}]
    with pytest.raises(TypeError, match="theta"):
        probe(rt, cos=cos, sin=sin, theta="1e6", start_position=7)
    with pytest.raises(TypeError, match="start_position"):
        probe(rt, cos=cos, sin=sin, theta=1e6, start_position=-1)
    with pytest.raises(ValueError, match="kind"):
        PushConstantInput("x", "float64")
