"""Decode parity harness: GPU greedy tokens against the CPU oracle decoder (TEST INFRASTRUCTURE ONLY).

Imported by tests/ and __graft_entry__.smoke() only.  Builds the CPU oracle model from the exact packed
bytes the GPU runs on (dequantized by the C oracle), then replays the GPU's tokens teacher-forced and
checks each one against the oracle's logits:

* if the oracle's top-2 margin exceeds ``tie_tol``, the GPU token must equal the oracle argmax;
* otherwise the GPU token's oracle logit must be within ``tie_tol`` of the maximum;
* the number of steps whose GPU token differs from the oracle argmax is bounded.

The exact-token rule is the reference's (token compares use equality, src/torch2vk/runtime/compare.py:119-128);
the oracle rounds the same tensors to bf16 as the kernels (matrix-product inputs, KV cache), so the near-tie
allowance covers only fp32 summation order and the bf16 roundings it can flip.
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
                        prompt_embeds: torch.Tensor | None = None, start: int = 0,
                        kv_init: tuple[torch.Tensor, torch.Tensor] | None = None,
                        max_mismatch: int | None = None, tie_tol_rms: float | None = None) -> dict:
    """Teacher-forced replay of ``gpu_tokens`` on the oracle; returns stats, raises AssertionError on mismatch.
    ``prompt_embeds`` [len(prompt), H] replaces the prompt's embedding lookup (injected audio features).
    ``kv_init`` (k, v) [layers, start, NK, D] fills cache positions 0..start-1 first (a prefilled KV cache); the
    prompt then runs at positions start..  The oracle stages matrix-product inputs and the KV cache in bf16 as the
    kernels do (``kv_bf16``), so the GPU's logits differ from it only by fp32 summation order.
    ``max_mismatch`` bounds the steps where the GPU token is not the oracle's argmax (allowed only inside
    the near-tie allowance); the default is one in ten steps, at least one.  ``tie_tol_rms`` makes the allowance
    scale with the step's logits: max(tie_tol, tie_tol_rms * rms(logits))."""
    n_pos = start + len(prompt) + len(gpu_tokens) + 1
    model = Qwen3CpuModel(shape, dense, max_positions=n_pos, stage_bf16=kv_bf16)
    if kv_init is not None:
        k0, v0 = kv_init
        assert k0.shape[1] == start and v0.shape[1] == start
        model.k_cache[:, :start] = k0.float()
        model.v_cache[:, :start] = v0.float()
    hidden = model.forward(torch.tensor(prompt), start=start, embeds=prompt_embeds)
    exact = 0
    near = 0
    mismatch = 0
    min_margin = float("inf")
    for i, tok in enumerate(gpu_tokens):
        logits = model.logits(hidden).double().numpy()
        order = np.argsort(-logits, kind="stable")
        best = int(order[0])
        margin = float(logits[order[0]] - logits[order[1]])
        min_margin = min(min_margin, margin)
        tol = tie_tol if tie_tol_rms is None else max(tie_tol, tie_tol_rms * float(np.sqrt(np.mean(logits ** 2))))
        if margin > tol:
            assert tok == best, f"step {i}: GPU token {tok} != oracle argmax {best} (margin {margin:.4g}, allowance {tol:.4g})"
            exact += 1
        else:
            assert logits[best] - logits[tok] <= tol, (
                f"step {i}: GPU token {tok} logit {logits[tok]:.5f} vs max {logits[best]:.5f}")
            near += 1
        mismatch += int(tok != best)
        if i + 1 < len(gpu_tokens):
            hidden = model.forward(torch.tensor([tok]), start=start + len(prompt) + i)
    bound = max(1, len(gpu_tokens) // 10) if max_mismatch is None else max_mismatch
    assert mismatch <= bound, f"{mismatch} of {len(gpu_tokens)} GPU tokens are not the oracle's argmax (bound {bound})"
    return {"exact": exact, "near_tie": near, "mismatch": mismatch, "min_margin": min_margin}


def oracle_step_logits(shape: Qwen3Shape, dense: dict[str, torch.Tensor], k_cache: torch.Tensor,
                       v_cache: torch.Tensor, token: int, position: int, *, stage_bf16: bool = True) -> np.ndarray:
    """The oracle's logits for ``token`` at ``position`` over a given KV history (rows 0..position-1 of every
    layer, [layers, position, NK, D], e.g. the GPU's own bf16 cache): one decode step, so a GPU step's logits can
    be held to a stated tolerance without the drift of a teacher-forced replay."""
    model = Qwen3CpuModel(shape, dense, max_positions=position + 1, stage_bf16=stage_bf16)
    model.k_cache[:, :position] = k_cache.float()
    model.v_cache[:, :position] = v_cache.float()
    hidden = model.forward(torch.tensor([token]), start=position)
    return model.logits(hidden).double().numpy()
