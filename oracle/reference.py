"""Reference math for the decode/prefill hot path (TEST INFRASTRUCTURE ONLY).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import this module.  Everything here runs on the CPU (numpy / torch
CPU) and is the checker for the HIP kernels, never the thing measured.

Each function names the reference code whose semantics it follows.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np
import torch

RMS_EPS = 1e-6  # rms_norm_mul_f16_f32.py:109 hard-codes 0.000001
F32_LOWEST = -3.4028234663852886e38


def bf16_round(x: np.ndarray) -> np.ndarray:
    """Round fp32 to bf16 (RNE) and return as fp32."""
    t = torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32))
    return t.to(torch.bfloat16).to(torch.float32).numpy()


def gemv_ref(x: np.ndarray, w_deq: np.ndarray) -> np.ndarray:
    """y = x . W^T in float64 (the LINEAR_NOBIAS_*_MATVEC contract, linear_nobias_q4_k_matvec_f32.py:26-61)."""
    return np.asarray(x, np.float64) @ np.asarray(w_deq, np.float64).T


def argmax_lowest(scores: np.ndarray) -> int:
    """Greedy select: highest score, ties to the lowest token id.

    better_pair in lm_head_q6_k_argmax_partial_f16.py:179-181 and
    qwen3_token_select_reduce_f32.py (subgroupMax then subgroupMin of tied ids).
    """
    scores = np.asarray(scores)
    best = scores.max()
    return int(np.flatnonzero(scores == best)[0])


def rms_norm(x: np.ndarray, weight: np.ndarray, eps: float = RMS_EPS) -> np.ndarray:
    """x * rsqrt(mean(x^2) + eps) * w over the last axis (rms_norm_mul_f16_f32.py:82-111)."""
    x = np.asarray(x, np.float64)
    inv = 1.0 / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)
    return x * inv * np.asarray(weight, np.float64)


def rope_cos_sin(positions: np.ndarray, head_dim: int, theta: float) -> tuple[np.ndarray, np.ndarray]:
    """cos/sin [T, D] with inv_freq = theta^(-2(d mod D/2)/D) (rope_table.py:105-119)."""
    half = head_dim // 2
    freq_idx = np.arange(head_dim) % half
    inv_freq = theta ** (-(2.0 * freq_idx) / head_dim)
    ang = np.asarray(positions, np.float64)[:, None] * inv_freq[None, :]
    return np.cos(ang), np.sin(ang)


def rotate_half(x: np.ndarray) -> np.ndarray:
    """rotate_half(x)[d] = -x[d+D/2] for d < D/2, x[d-D/2] otherwise (rms_norm_rope_transpose_f16.py:133-143)."""
    half = x.shape[-1] // 2
    return np.concatenate([-x[..., half:], x[..., :half]], axis=-1)


def qk_norm_rope(x: np.ndarray, weight: np.ndarray, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    """Per-head RMSNorm over D then rotate-half RoPE (RMS_NORM_ROPE_TRANSPOSE_F16)."""
    n = rms_norm(x, weight)
    return n * cos + rotate_half(n) * sin


def silu_mul(gate: np.ndarray, up: np.ndarray) -> np.ndarray:
    """silu(gate) * up (swiglu_f16.py:74-77)."""
    g = np.asarray(gate, np.float64)
    return g / (1.0 + np.exp(-g)) * np.asarray(up, np.float64)


def attention_ref(q: np.ndarray, k: np.ndarray, v: np.ndarray, *, causal_offset: int | None = None,
                  mask: np.ndarray | None = None) -> np.ndarray:
    """softmax(q k^T / sqrt(D) [+ mask]) v with GQA head mapping kv_head = head*NK/NH.

    q [T, NH, D]; k, v [S, NK, D].  ``causal_offset`` c lets query row t see keys <= c + t.
    Follows sdpa_decode_cache_write_f32.py:104-168 (decode) and sdpa_causal_f32.py (prefill).
    """
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    t_len, nh, d = q.shape
    s_len, nk, _ = k.shape
    out = np.zeros((t_len, nh, d))
    for h in range(nh):
        kvh = h * nk // nh
        scores = q[:, h, :] @ k[:, kvh, :].T / math.sqrt(d)
        if mask is not None:
            scores = scores + mask
        if causal_offset is not None:
            allowed = np.arange(s_len)[None, :] <= (causal_offset + np.arange(t_len))[:, None]
            scores = np.where(allowed, scores, -np.inf)
        scores = scores - scores.max(axis=-1, keepdims=True)
        p = np.exp(scores)
        p = p / p.sum(axis=-1, keepdims=True)
        out[:, h, :] = p @ v[:, kvh, :]
    return out


# --------------------------------------------------------------------------
# Qwen3 decoder on the CPU (torch), used for token parity and as the CPU
# baseline.  Semantics follow HF Qwen3 as exported by the reference
# (src/models/quantized_qwen3/export.py:102-119): pre-norm blocks, per-head
# q/k RMSNorm, rotate-half RoPE, GQA, SwiGLU MLP, final norm, untied LM head.
# --------------------------------------------------------------------------


@dataclass(frozen=True)
class Qwen3Shape:
    hidden: int
    layers: int
    heads: int
    kv_heads: int
    head_dim: int
    mlp: int
    vocab: int
    rope_theta: float = 1.0e6


class Qwen3CpuModel:
    """Dense CPU Qwen3 over already-dequantized weights.

    ``weights`` maps names to float tensors: ``embed`` [V,H], ``lm_head`` [V,H],
    ``norm`` [H] and per layer ``layers.{i}.{q,k,v,o,gate,up,down}`` plus
    ``layers.{i}.{input_norm,post_norm,q_norm,k_norm}``.
    """

    def __init__(self, shape: Qwen3Shape, weights: dict[str, torch.Tensor], max_positions: int,
                 dtype: torch.dtype = torch.float32, stage_bf16: bool = False) -> None:
        self.shape = shape
        self.dtype = dtype
        # stage_bf16: round every matrix-product input to bf16 and keep K/V in bf16, as the decode kernels
        # stage them (RMSNorm output, attention output, SwiGLU output, the LM head input and the KV cache);
        # the residual stream, q and the products stay fp32.  The reference stages the same tensors in fp16
        # (src/torch2vk/export/dtype_policy.py:23-36).
        self.stage_bf16 = stage_bf16
        self.w = {k: v.to(dtype) for k, v in weights.items()}
        s = shape
        self.k_cache = torch.zeros(s.layers, max_positions, s.kv_heads, s.head_dim, dtype=dtype)
        self.v_cache = torch.zeros_like(self.k_cache)
        half = s.head_dim // 2
        freq_idx = torch.arange(s.head_dim, dtype=torch.float64) % half
        self.inv_freq = s.rope_theta ** (-(2.0 * freq_idx) / s.head_dim)

    @staticmethod
    def _rms(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
        xf = x.to(torch.float32)
        inv = torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + RMS_EPS)
        return (xf * inv).to(x.dtype) * w

    def _stage(self, x: torch.Tensor) -> torch.Tensor:
        return x.to(torch.bfloat16).to(x.dtype) if self.stage_bf16 else x

    def _rope(self, x: torch.Tensor, positions: torch.Tensor) -> torch.Tensor:
        ang = positions.to(torch.float64)[:, None] * self.inv_freq[None, :]
        cos = torch.cos(ang).to(x.dtype)[:, None, :]
        sin = torch.sin(ang).to(x.dtype)[:, None, :]
        half = x.shape[-1] // 2
        rot = torch.cat([-x[..., half:], x[..., :half]], dim=-1)
        return x * cos + rot * sin

    def forward(self, tokens: torch.Tensor, start: int, layers: int | None = None,
                embeds: torch.Tensor | None = None, mask: torch.Tensor | None = None,
                all_positions: bool = False) -> torch.Tensor:
        """Run T tokens at positions start..start+T-1, fill the KV cache, return last hidden [H] (post final norm).
        ``embeds`` [T, H] replaces the embedding lookup (a prompt with injected audio features).  ``mask``: an
        additive fp32 [T, start + T] attention mask used instead of the causal one (OmniVoice's LLM pass,
        src/models/quantized_omnivoice/dispatch/llm_forward.py:19-70 with SDPA_MASKED_F32); ``all_positions``
        returns every position's final-normed hidden [T, H] (that pass's output, llm_forward.py:70)."""
        s = self.shape
        w = self.w
        t_len = tokens.shape[0] if embeds is None else embeds.shape[0]
        positions = torch.arange(start, start + t_len)
        h = w["embed"][tokens] if embeds is None else embeds.to(self.dtype)
        group = s.heads // s.kv_heads
        n_layers = s.layers if layers is None else layers
        for i in range(n_layers):
            p = f"layers.{i}."
            x = self._stage(self._rms(h, w[p + "input_norm"]))
            q = (x @ w[p + "q"].T).view(t_len, s.heads, s.head_dim)
            k = (x @ w[p + "k"].T).view(t_len, s.kv_heads, s.head_dim)
            v = (x @ w[p + "v"].T).view(t_len, s.kv_heads, s.head_dim)
            q = self._rope(self._rms(q, w[p + "q_norm"]), positions)
            k = self._rope(self._rms(k, w[p + "k_norm"]), positions)
            self.k_cache[i, start:start + t_len] = self._stage(k)
            self.v_cache[i, start:start + t_len] = self._stage(v)
            keys = self.k_cache[i, :start + t_len].repeat_interleave(group, dim=1)
            vals = self.v_cache[i, :start + t_len].repeat_interleave(group, dim=1)
            scores = torch.einsum("thd,shd->hts", q.float(), keys.float()) / math.sqrt(s.head_dim)
            if mask is None:
                allowed = torch.arange(start + t_len)[None, :] <= positions[:, None]
                scores = scores.masked_fill(~allowed[None], float("-inf"))
            else:
                scores = scores + mask.float()[None]
            probs = torch.softmax(scores, dim=-1)
            attn = torch.einsum("hts,shd->thd", probs, vals.float()).to(self.dtype).reshape(t_len, -1)
            h = h + self._stage(attn) @ w[p + "o"].T
            x = self._stage(self._rms(h, w[p + "post_norm"]))
            g = x @ w[p + "gate"].T
            u = x @ w[p + "up"].T
            h = h + self._stage(torch.nn.functional.silu(g) * u) @ w[p + "down"].T
        return self._rms(h, w["norm"]) if all_positions else self._rms(h[-1], w["norm"])

    def logits(self, hidden: torch.Tensor) -> torch.Tensor:
        return self._stage(hidden) @ self.w["lm_head"].T
