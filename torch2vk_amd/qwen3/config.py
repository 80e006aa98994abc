"""Qwen3 decoder shapes and the GGUF type policy.

The reference ships Qwen3-0.6B only (src/models/quantized_qwen3/export_gguf.py:15); its kernels are
shape-symbolic, so the 8B is the same path at other N/K.
"""

from __future__ import annotations

from dataclasses import dataclass


@dataclass(frozen=True)
class Qwen3Config:
    name: str
    hidden: int
    layers: int
    heads: int
    kv_heads: int
    head_dim: int
    mlp: int
    vocab: int
    rope_theta: float = 1.0e6
    rms_eps: float = 1.0e-6
    eos_token_ids: tuple[int, ...] = (151645,)

    @property
    def q_dim(self) -> int:
        return self.heads * self.head_dim

    @property
    def kv_dim(self) -> int:
        return self.kv_heads * self.head_dim


QWEN3_0_6B = Qwen3Config("qwen3-0.6b", hidden=1024, layers=28, heads=16, kv_heads=8, head_dim=128, mlp=3072,
                         vocab=151936)
QWEN3_1_7B = Qwen3Config("qwen3-1.7b", hidden=2048, layers=28, heads=16, kv_heads=8, head_dim=128, mlp=6144,
                         vocab=151936)
QWEN3_8B = Qwen3Config("qwen3-8b", hidden=4096, layers=36, heads=32, kv_heads=8, head_dim=128, mlp=12288,
                       vocab=151936)


def q4_k_m_more_bits_layer_indices(num_layers: int) -> tuple[int, ...]:
    """Layers whose v_proj/down_proj get Q6_K under Q4_K_M (src/torch2vk/quantize/gguf.py:150-161)."""
    if num_layers <= 0:
        raise ValueError(f"num_layers must be positive, got {num_layers}")
    first_eighth = num_layers // 8
    last_eighth = (7 * num_layers) // 8
    return tuple(i for i in range(num_layers)
                 if i < first_eighth or i >= last_eighth or (i - first_eighth) % 3 == 2)


def gguf_type(shape: tuple[int, ...], *, force_q6: bool = False, force_q8: bool = False) -> str:
    """Per-tensor type rule of Q4KMQuantizationConfig.gguf_type (src/torch2vk/quantize/gguf.py:54-83)."""
    if force_q8 and len(shape) >= 2:
        return "q8_0"
    if force_q6 and len(shape) >= 2:
        return "q6_k"
    if len(shape) != 2:
        return "f32"
    cols = shape[-1]
    if cols % 256 == 0:
        return "q4_k"
    if cols % 32 == 0:
        return "q8_0"
    return "f32"


def tensor_types(config: Qwen3Config, policy: str) -> dict[str, str]:
    """GGUF type of every 2-D weight under ``policy``: "uniform" int4, "q4_k_m", or "qwen3_asr" (Q4_K_M with
    the token embedding forced to Q8_0, the Qwen3-ASR thinker's rule: src/models/quantized_qwen3_asr/
    quantization.py:8,24-32)."""
    if policy not in ("uniform", "q4_k_m", "qwen3_asr"):
        raise ValueError(f"unknown policy {policy!r}")
    km = policy in ("q4_k_m", "qwen3_asr")
    more_bits = set(q4_k_m_more_bits_layer_indices(config.layers)) if km else set()
    c = config
    types = {
        "embed": gguf_type((c.vocab, c.hidden), force_q8=policy == "qwen3_asr"),
        "lm_head": gguf_type((c.vocab, c.hidden), force_q6=km),
    }
    for i in range(c.layers):
        p = f"layers.{i}."
        types[p + "q"] = gguf_type((c.q_dim, c.hidden))
        types[p + "k"] = gguf_type((c.kv_dim, c.hidden))
        types[p + "v"] = gguf_type((c.kv_dim, c.hidden), force_q6=i in more_bits)
        types[p + "o"] = gguf_type((c.hidden, c.q_dim))
        types[p + "gate"] = gguf_type((c.mlp, c.hidden))
        types[p + "up"] = gguf_type((c.mlp, c.hidden))
        types[p + "down"] = gguf_type((c.hidden, c.mlp), force_q6=i in more_bits)
    return types
