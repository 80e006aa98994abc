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
