"""Decode parity harness: GPU greedy tokens against the CPU oracle decoder (TEST INFRASTRUCTURE ONLY).

Imported by tests/ and __graft_entry__.smoke() only.  Builds the CPU oracle model from the exact packed
bytes the GPU runs on (dequantized by the C oracle), then replays the GPU's tokens teacher-forced and
checks each one against the oracle's logits:

* if the oracle's top-2 margin exceeds ``tie_tol``, the GPU token must equal the oracle argmax;
* otherwise the GPU token's oracle logit must be within ``tie_tol`` of the maximum.

The exact-token rule is the reference's (token compares use equality, src/torch2vk/runtime/compare.py:119-128);
the near-tie allowance covers bf16 activation rounding, which the fp32 oracle does not perform.
"""

from __future__ import annotations

import numpy as np
import torch

from oracle import quant
from oracle.reference import Qwen3CpuModel, Qwen3Shape


def dense_weights(packed: dict[str, np.ndarray], types: dict[str, str], norms: dict[str, np.ndarray],
                  shapes: dict[str, tuple[int, int]]) -> dict[str, torch.Tensor]:
    out = {}
    for name, arr in packed.items():
        rows, k = shapes[name]
        t = types[name]
        if t == "q4_k":
            d = quant.dequant_q4_k(arr, k)
        elif t == "q6_k":
            d = quant.dequant_q6_k(arr, k)
        elif t == "q8_0":
            d = quant.dequant_q8_0(arr, k)
        else:
            raise ValueError(f"{name}: unsupported type {t}")
        assert d.shape == (rows, k)
        out[name] = torch.from_numpy(d)
    for name, arr in norms.items():
        out[name] = torch.from_numpy(np.asarray(arr, np.float32))
    return out


def check_greedy_tokens(shape: Qwen3Shape, dense: dict[str, torch.Tensor], prompt: list[int], gpu_tokens: list[int],
                        *, tie_tol: float = 5e-3, kv_bf16: bool = True,
                        prompt_embeds: torch.Tensor | None = None) -> dict:
    """Teacher-forced replay of ``gpu_tokens`` on the oracle; returns stats, raises AssertionError on mismatch.
    ``prompt_embeds`` [len(prompt), H] replaces the prompt's embedding lookup (injected audio features)."""
    model = Qwen3CpuModel(shape, dense, max_positions=len(prompt) + len(gpu_tokens) + 1)
    hidden = model.forward(torch.tensor(prompt), start=0, embeds=prompt_embeds)
    exact = 0
    near = 0
    min_margin = float("inf")
    for i, tok in enumerate(gpu_tokens):
        logits = model.logits(hidden).double().numpy()
        order = np.argsort(-logits, kind="stable")
        best = int(order[0])
        margin = float(logits[order[0]] - logits[order[1]])
        min_margin = min(min_margin, margin)
        if margin > tie_tol:
            assert tok == best, f"step {i}: GPU token {tok} != oracle argmax {best} (margin {margin:.4g})"
            exact += 1
        else:
            assert logits[best] - logits[tok] <= tie_tol, (
                f"step {i}: GPU token {tok} logit {logits[tok]:.5f} vs max {logits[best]:.5f}")
            near += 1
        if i + 1 < len(gpu_tokens):
            if kv_bf16:
                model.k_cache.copy_(model.k_cache.to(torch.bfloat16).float())
                model.v_cache.copy_(model.v_cache.to(torch.bfloat16).float())
            hidden = model.forward(torch.tensor([tok]), start=len(prompt) + i)
    return {"exact": exact, "near_tie": near, "min_margin": min_margin}
