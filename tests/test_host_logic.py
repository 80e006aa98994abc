"""Host-side logic: the GGUF type policy and model shapes (CPU only)."""

from __future__ import annotations

import pytest

from torch2vk_amd.qwen3.config import (
    QWEN3_0_6B,
    QWEN3_8B,
    gguf_type,
    q4_k_m_more_bits_layer_indices,
    tensor_types,
)
from torch2vk_amd.qwen3.weights import matrix_shapes, norm_shapes


def test_more_bits_layers_match_the_q4_k_m_rule():
    # i < L/8, i >= 7L/8, or (i - L/8) % 3 == 2 (src/torch2vk/quantize/gguf.py:150-161)
    assert q4_k_m_more_bits_layer_indices(28) == (0, 1, 2, 5, 8, 11, 14, 17, 20, 23, 24, 25, 26, 27)
    assert len(q4_k_m_more_bits_layer_indices(36)) == 18
    assert q4_k_m_more_bits_layer_indices(1) == (0,)
    with pytest.raises(ValueError):
        q4_k_m_more_bits_layer_indices(0)


def test_gguf_type_rule():
    assert gguf_type((4096, 4096)) == "q4_k"
    assert gguf_type((4096, 1056)) == "q8_0"       # K % 256 != 0 but K % 32 == 0
    assert gguf_type((4096, 1000)) == "f32"
    assert gguf_type((4096,)) == "f32"
    assert gguf_type((151936, 4096), force_q6=True) == "q6_k"
    assert gguf_type((10, 64), force_q8=True) == "q8_0"


def test_tensor_types_per_policy():
    uni = tensor_types(QWEN3_8B, "uniform")
    assert set(uni.values()) == {"q4_k"}
    km = tensor_types(QWEN3_0_6B, "q4_k_m")
    assert km["lm_head"] == "q6_k"
    assert km["layers.0.v"] == "q6_k" and km["layers.3.v"] == "q4_k" and km["layers.5.down"] == "q6_k"
    assert sum(t == "q6_k" for t in km.values()) == 1 + 2 * 14
    with pytest.raises(ValueError):
        tensor_types(QWEN3_8B, "q2")


def test_8b_byte_budget():
    """Packed bytes per decode token at uniform Q4_K: the roofline figure the bench reports against."""
    shapes = matrix_shapes(QWEN3_8B)
    per_layer = sum(r * c for n, (r, c) in shapes.items() if n.startswith("layers.0."))
    layers = QWEN3_8B.layers * per_layer * 144 // 256
    lm = 151936 * 4096 * 144 // 256
    assert layers == 3_906_994_176 and lm == 350_060_544
    assert len(norm_shapes(QWEN3_8B)) == 1 + 4 * 36


def _fake_layer_weights(types):
    """CPU stand-ins with the byte sizes of one Qwen3-0.6B-shape layer's packed weights (content unused), q|k
    (and a Q4_K v) stacked in one allocation as the weight loaders leave them."""
    import torch

    from torch2vk_amd.qwen3.config import QWEN3_0_6B as c
    row = {"q4_k": c.hidden // 256 * 144, "q6_k": c.hidden // 256 * 210}
    stacked = ["q", "k"] + (["v"] if types["layers.0.v"] == "q4_k" else [])
    n_rows = {"q": c.q_dim, "k": c.kv_dim, "v": c.kv_dim}
    fused = torch.zeros(sum(n_rows[n] for n in stacked) * row["q4_k"], dtype=torch.uint8)
    packed, begin = {}, 0
    for n in stacked:
        size = n_rows[n] * row["q4_k"]
        packed[f"layers.0.{n}"] = fused[begin:begin + size]
        begin += size
    if "layers.0.v" not in packed:
        packed["layers.0.v"] = torch.zeros(c.kv_dim * row["q6_k"], dtype=torch.uint8)
    for n in ("o", "gate", "up", "down"):
        packed[f"layers.0.{n}"] = torch.zeros(1, dtype=torch.uint8)
    norms = {f"layers.0.{n}": torch.ones(4) for n in ("input_norm", "post_norm", "q_norm", "k_norm")}
    cache = torch.zeros(1, 8, 8, 128, dtype=torch.bfloat16)
    return packed, norms, cache


@pytest.mark.parametrize("v,down,bits", [("q4_k", "q4_k", 0), ("q6_k", "q4_k", 1), ("q4_k", "q6_k", 2),
                                         ("q6_k", "q6_k", 3)])
def test_decode_layer_table_weight_types(v, down, bits):
    """The persistent kernel's table: 13 pointers, then bit 0 = Q6_K v, bit 1 = Q6_K down."""
    from torch2vk_amd import kernels

    types = {f"layers.0.{n}": "q4_k" for n in ("q", "k", "o", "gate", "up")}
    types["layers.0.v"], types["layers.0.down"] = v, down
    packed, norms, cache = _fake_layer_weights(types)
    table = kernels.decode_layer_table(packed, norms, 1, cache, cache, types)
    assert tuple(table.shape) == (1, kernels.DECODE_LAYER_TABLE_COLUMNS) == (1, 14)
    assert int(table[0, 13]) == bits
    assert int(table[0, 2]) == packed["layers.0.v"].data_ptr()
    assert int(table[0, 6]) == packed["layers.0.down"].data_ptr()


def test_decode_layer_table_rejects_other_layouts():
    from torch2vk_amd import kernels

    types = {f"layers.0.{n}": "q4_k" for n in ("q", "k", "v", "o", "gate", "up", "down")}
    packed, norms, cache = _fake_layer_weights(types)
    with pytest.raises(ValueError, match="o must be Q4_K"):
        kernels.decode_layer_table(packed, norms, 1, cache, cache, {**types, "layers.0.o": "q6_k"})
    with pytest.raises(ValueError, match="down must be Q4_K or Q6_K"):
        kernels.decode_layer_table(packed, norms, 1, cache, cache, {**types, "layers.0.down": "q8_0"})
    # a Q4_K v that is not stacked after k
    apart = dict(packed)
    apart["layers.0.v"] = apart["layers.0.v"].clone()
    with pytest.raises(ValueError, match="must follow k"):
        kernels.decode_layer_table(apart, norms, 1, cache, cache, types)
    apart = dict(packed)
    apart["layers.0.k"] = apart["layers.0.k"].clone()
    with pytest.raises(ValueError, match="q and k rows must be stacked"):
        kernels.decode_layer_table(apart, norms, 1, cache, cache, types)


@pytest.mark.parametrize("v_type", ["q4_k", "q6_k"])
def test_stack_qkv_keeps_q_and_k_together(v_type):
    """q and k rows share one allocation whatever v's type; v joins them only when it is Q4_K too."""
    import torch

    from dataclasses import replace
    from torch2vk_amd.qwen3.config import QWEN3_0_6B
    from torch2vk_amd.qwen3.weights import Qwen3Weights, stack_qkv

    cfg = replace(QWEN3_0_6B, layers=1)
    w = Qwen3Weights(config=cfg, policy="q4_k_m", types={"layers.0.q": "q4_k", "layers.0.k": "q4_k",
                                                         "layers.0.v": v_type})
    for n, rows in (("q", cfg.q_dim), ("k", cfg.kv_dim), ("v", cfg.kv_dim)):
        w.packed[f"layers.0.{n}"] = torch.full((rows, 8), len(n), dtype=torch.uint8)
    before = {n: t.clone() for n, t in w.packed.items()}
    stack_qkv(w)
    q, k, v = (w.packed[f"layers.0.{n}"] for n in ("q", "k", "v"))
    assert k.data_ptr() == q.data_ptr() + q.numel()
    assert (v.data_ptr() == k.data_ptr() + k.numel()) == (v_type == "q4_k")
    for n, t in before.items():
        assert torch.equal(w.packed[n], t)
