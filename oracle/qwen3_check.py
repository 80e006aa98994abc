"""Decode parity harness: GPU greedy tokens against the CPU oracle decoder (TEST INFRASTRUCTURE ONLY).

Imported by tests/ and __graft_entry__.smoke() only.  Builds the CPU oracle model from the exact packed
bytes the GPU runs on (dequantized by the C oracle), then replays the GPU's tokens teacher-forced.  Token ids
compare by equality, as the reference's compares do (src/torch2vk/runtime/compare.py:119-128).  There is no
near-tie allowance.  A step whose GPU token is not the replay's argmax must be explained by one of:

* drift of the replay's own KV history: the oracle's logits for that step over the GPU's own cache rows
  (one step, ``oracle_step_logits``) have the GPU token as their lowest-id argmax;
* the step's own rounding: the GPU's logits for that step (re-run on the GPU, ``gpu_logits``) have the GPU token
  as their lowest-id argmax, and lie within the per-step tolerance (max-abs ``step_tol_rms`` of the logits' rms)
  of the oracle's over the same history.

The oracle rounds the same tensors to bf16 as the kernels (matrix-product inputs, KV cache), so what remains
between the two is fp32 summation order and the bf16 roundings it can flip.
"""

from __future__ import annotations

from typing import Callable

import numpy as np
import torch

from oracle import quant
from oracle.reference import Qwen3CpuModel, Qwen3Shape, argmax_lowest

# Per-step logits tolerance: max-abs error as a fraction of the logits' rms, for one decode step over a given KV
# history.  Measured 1.4e-2 .. 2.5e-2 at 4 layers and 1.5e-2 at 28 layers (bf16 staging of activations; one that
# lands on the other side of a bf16 rounding boundary moves by 2^-8 of itself).
STEP_TOL_RMS = 3e-2

GpuLogits = Callable[[int, int, "int | None", "torch.Tensor | None"], np.ndarray]


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


def decoder_step_logits(dec, prefill_h: torch.Tensor | None = None) -> GpuLogits:
    """``gpu_logits`` for check_greedy_tokens over a decoder object with ``step_logits(position, token=, embed=)``
    and ``logits(h)`` methods.  ``prefill_h``: the residual row a chunked prefill ended with (step 0's token was
    selected from it, not from a decode step)."""
    def fn(step: int, position: int, token: int | None, embed: torch.Tensor | None) -> np.ndarray:
        if step == 0 and prefill_h is not None:
            out = dec.logits(prefill_h)
        elif embed is not None:
            out = dec.step_logits(position, embed=embed.to(device=dec.device, dtype=torch.float32))
        else:
            out = dec.step_logits(position, token=token)
        return out.float().cpu().numpy()
    return fn


def check_greedy_tokens(shape: Qwen3Shape, dense: dict[str, torch.Tensor], prompt: list[int], gpu_tokens: list[int],
                        *, kv_history: tuple[torch.Tensor, torch.Tensor] | None = None,
                        gpu_logits: GpuLogits | None = None, step_tol_rms: float = STEP_TOL_RMS,
                        kv_bf16: bool = True, prompt_embeds: torch.Tensor | None = None, start: int = 0,
                        kv_init: tuple[torch.Tensor, torch.Tensor] | None = None, label: str = "") -> dict:
    """Teacher-forced replay of ``gpu_tokens`` on the oracle; returns counts, raises AssertionError on a step the
    rules above do not explain.  ``kv_history`` (k, v) [layers, >= positions, NK, D] (any device): the GPU's KV
    cache after the run, whose rows 0..p-1 are the history of the step at position p.  ``gpu_logits(step,
    position, token, embed)``: the GPU's fp32 logits of a step (``decoder_step_logits``).  ``prompt_embeds``
    [len(prompt), H] replaces the prompt's embedding lookup (injected audio features).  ``kv_init`` (k, v)
    [layers, start, NK, D] fills cache positions 0..start-1 first (a prefilled KV cache); the prompt then runs at
    positions start.."""
    n_pos = start + len(prompt) + len(gpu_tokens) + 1
    model = Qwen3CpuModel(shape, dense, max_positions=n_pos, stage_bf16=kv_bf16)
    if kv_init is not None:
        k0, v0 = kv_init
        assert k0.shape[1] == start and v0.shape[1] == start
        model.k_cache[:, :start] = k0.float()
        model.v_cache[:, :start] = v0.float()
    hidden = model.forward(torch.tensor(prompt), start=start, embeds=prompt_embeds)
    counts = {"steps": len(gpu_tokens), "exact": 0, "history": 0, "near": 0}
    min_margin = float("inf")
    worst = 0.0
    first = start + len(prompt) - 1
    for i, tok in enumerate(gpu_tokens):
        logits = model.logits(hidden).double().numpy()
        order = np.argsort(-logits, kind="stable")
        margin = float(logits[order[0]] - logits[order[1]])
        min_margin = min(min_margin, margin)
        best = argmax_lowest(logits)
        if tok == best:
            counts["exact"] += 1
        else:
            pos = first + i
            token_in = prompt[-1] if i == 0 else gpu_tokens[i - 1]
            embed = prompt_embeds[-1] if (i == 0 and prompt_embeds is not None) else None
            where = f"{label} step {i} (position {pos}): GPU token {tok}, replay argmax {best} (margin {margin:.4g})"
            assert kv_history is not None, f"{where}: no GPU KV history to check the step on ({counts})"
            k_hist, v_hist = kv_history
            ref = oracle_step_logits(shape, dense, k_hist[:, :pos].float().cpu(), v_hist[:, :pos].float().cpu(),
                                     None if embed is not None else token_in, pos, embed=embed, stage_bf16=kv_bf16)
            best_h = argmax_lowest(ref)
            if best_h == tok:
                counts["history"] += 1
                print(f"{where}: the oracle over the GPU's KV history picks {tok} (its gap to {best} "
                      f"{ref[tok] - ref[best]:.4g})", flush=True)
            else:
                assert gpu_logits is not None, f"{where}: oracle over the GPU history picks {best_h} ({counts})"
                got = np.asarray(gpu_logits(i, pos, None if embed is not None else token_in, embed), np.float64)
                rms = float(np.sqrt(np.mean(ref * ref)))
                err = float(np.abs(got - ref).max())
                worst = max(worst, err / rms)
                gpu_best = argmax_lowest(got.astype(np.float32))
                print(f"{where}: oracle over the GPU history picks {best_h} (gap {ref[best_h] - ref[tok]:.4g}); "
                      f"GPU logits max-abs {err:.4g} = {err / rms:.3g} of rms {rms:.4g}, GPU argmax {gpu_best}",
                      flush=True)
                assert gpu_best == tok, f"{where}: the GPU's own logits pick {gpu_best} ({counts})"
                assert err <= step_tol_rms * rms, (f"{where}: GPU logits max-abs {err:.4g} > {step_tol_rms} of "
                                                   f"rms {rms:.4g} ({counts})")
                counts["near"] += 1
        if i + 1 < len(gpu_tokens):
            hidden = model.forward(torch.tensor([tok]), start=first + 1 + i)
    counts["min_margin"] = min_margin
    if worst:
        counts["worst_step_err_rms"] = worst
    return counts


def oracle_step_logits(shape: Qwen3Shape, dense: dict[str, torch.Tensor], k_cache: torch.Tensor,
                       v_cache: torch.Tensor, token: int | None, position: int, *, embed: torch.Tensor | None = None,
                       stage_bf16: bool = True) -> np.ndarray:
    """The oracle's logits for ``token`` (or the input row ``embed``) at ``position`` over a given KV history
    (rows 0..position-1 of every layer, [layers, position, NK, D], e.g. the GPU's own bf16 cache): one decode
    step, so a GPU step's logits can be held to a stated tolerance without the drift of a teacher-forced
    replay."""
    model = Qwen3CpuModel(shape, dense, max_positions=position + 1, stage_bf16=stage_bf16)
    model.k_cache[:, :position] = k_cache.float()
    model.v_cache[:, :position] = v_cache.float()
    if embed is None:
        hidden = model.forward(torch.tensor([token]), start=position)
    else:
        hidden = model.forward(None, start=position, embeds=embed.float().cpu().reshape(1, -1))
    return model.logits(hidden).double().numpy()
