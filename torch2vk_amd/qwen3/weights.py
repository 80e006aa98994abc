"""Synthetic random-init Qwen3 weights, quantized on the GPU.

There is no checkpoint to load offline, so the decoder runs on seeded
N(0, std) weights, drawn on the device and packed into GGUF
blocks by the GPU quantizers (bit-identical to the reference quantizer as
restated in the CPU oracle).  Draw order is fixed: embed, then per layer
q, k, v, o, gate, up, down, then lm_head, then the norm weights.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import torch

from torch2vk_amd import kernels
from torch2vk_amd.qwen3.config import Qwen3Config, tensor_types


def matrix_shapes(c: Qwen3Config) -> dict[str, tuple[int, int]]:
    shapes = {"embed": (c.vocab, c.hidden)}
    for i in range(c.layers):
        p = f"layers.{i}."
        shapes[p + "q"] = (c.q_dim, c.hidden)
        shapes[p + "k"] = (c.kv_dim, c.hidden)
        shapes[p + "v"] = (c.kv_dim, c.hidden)
        shapes[p + "o"] = (c.hidden, c.q_dim)
        shapes[p + "gate"] = (c.mlp, c.hidden)
        shapes[p + "up"] = (c.mlp, c.hidden)
        shapes[p + "down"] = (c.hidden, c.mlp)
    shapes["lm_head"] = (c.vocab, c.hidden)
    return shapes


def norm_shapes(c: Qwen3Config) -> dict[str, int]:
    shapes = {"norm": c.hidden}
    for i in range(c.layers):
        p = f"layers.{i}."
        shapes[p + "input_norm"] = c.hidden
        shapes[p + "post_norm"] = c.hidden
        shapes[p + "q_norm"] = c.head_dim
        shapes[p + "k_norm"] = c.head_dim
    return shapes


@dataclass
class Qwen3Weights:
    config: Qwen3Config
    policy: str
    packed: dict[str, torch.Tensor] = field(default_factory=dict)   # uint8 GGUF rows
    types: dict[str, str] = field(default_factory=dict)             # "q4_k" | "q6_k" | "q8_0"
    norms: dict[str, torch.Tensor] = field(default_factory=dict)    # fp32

    def packed_bytes(self, names=None) -> int:
        names = self.packed.keys() if names is None else names
        return sum(self.packed[n].numel() for n in names)


def synthetic_weights(config: Qwen3Config, *, device, seed: int = 0, std: float = 0.02, norm_std: float = 0.0,
                      policy: str = "uniform") -> Qwen3Weights:
    """Seeded N(0, std) weights quantized per ``policy``; norm weights 1 + N(0, norm_std)."""
    types = tensor_types(config, policy)
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    w = Qwen3Weights(config=config, policy=policy, types=types)
    for name, (rows, cols) in matrix_shapes(config).items():
        dense = torch.randn(rows, cols, generator=gen, device=device, dtype=torch.float32).mul_(std)
        w.packed[name] = kernels.quantize(dense, types[name])
        del dense
    stack_qkv(w)
    for name, n in norm_shapes(config).items():
        t = torch.ones(n, dtype=torch.float32, device=device)
        if norm_std > 0:
            t.add_(torch.randn(n, generator=gen, device=device, dtype=torch.float32).mul_(norm_std))
        w.norms[name] = t
    return w


def stack_qkv(w: Qwen3Weights) -> None:
    """Keep each layer's q and k rows, and v's when it has their GGUF type, in one allocation (they become
    views of it): the persistent decode kernel streams them as one matrix (6144 rows at the 8B shape), and
    a Q6_K v (Q4_K_M more-bits layers) as its own.  Rows are quantized independently, so the bytes are
    unchanged."""
    for i in range(w.config.layers):
        names = [f"layers.{i}.{n}" for n in ("q", "k", "v")]
        if w.types[names[0]] != w.types[names[1]]:
            continue
        if w.types[names[2]] != w.types[names[0]]:
            names = names[:2]
        parts = [w.packed[n] for n in names]
        fused = torch.cat(parts, dim=0)
        begin = 0
        for n, t in zip(names, parts):
            w.packed[n] = fused[begin:begin + t.shape[0]]
            begin += t.shape[0]
