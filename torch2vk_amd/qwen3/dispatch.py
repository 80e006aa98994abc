"""Qwen3 decode layer as the reference's dispatch function: run_decode_layer(rt, layer_idx, *, cache_position).

Mirrors src/models/optimized_qwen3/dispatch/decode_layer.py:22-136: the layer's tensors come from the bound
model tensors (``model_tensors().decode_layers[layer_idx]``), and the layer is a sequence of variant calls, each
checked against its contract by ``rt.dispatch``:

    RMS_NORM_MUL_F16_F32                        input RMSNorm
    LINEAR_NOBIAS_Q4_K_QKV_MATVEC_F32           q|k|v (LINEAR_NOBIAS_Q4_QK_Q6_V_MATVEC_F32 for a Q6_K v)
    SDPA_DECODE_QK_NORM_ROPE_CACHE_WRITE_F32    q/k RMSNorm + RoPE + KV write + attention (the reference's
                                                RMS_NORM_ROPE_TRANSPOSE_F16 x2 + SDPA_DECODE_CACHE_WRITE_F32)
    LINEAR_NOBIAS_Q{4,6}_K_MATVEC_ADD_F32       o_proj + residual
    RMS_NORM_MUL_F16_F32                        post-attention RMSNorm
    LINEAR_NOBIAS_Q4_K_QK_MATVEC_F32            gate|up
    SWIGLU_F16
    LINEAR_NOBIAS_Q{4,6}_K_MATVEC_ADD_F32       down + residual

Weights are the decoder's packed GGUF rows viewed as the reference's physical types (Q4_K uint32 words, Q6_K
uint16 halfwords) without a copy.  This is the reference-named surface; Qwen3Decoder runs the same arithmetic
with fewer launches (RMSNorm fused into the GEMV prologues) or in one persistent launch.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from torch2vk_amd import variants as V
from torch2vk_amd.runtime import RuntimeSession


@dataclass
class DecodeLayerTensors:
    """One layer's tensors in the reference's roles (src/models/optimized_qwen3/tensors/decode_layer.py)."""
    hidden: torch.Tensor                 # fp32 [1, 1, H], the residual stream (read and updated in place)
    normed: torch.Tensor                 # bf16 [1, 1, H]
    q: torch.Tensor                      # fp32 [1, 1, NQ]
    k: torch.Tensor                      # fp32 [1, 1, NKV]
    v: torch.Tensor                      # fp32 [1, 1, NKV]
    attn: torch.Tensor                   # bf16 [1, NH, 1, D]
    gate: torch.Tensor                   # fp32 [1, 1, MLP]
    up: torch.Tensor                     # fp32 [1, 1, MLP]
    act: torch.Tensor                    # bf16 [1, 1, MLP]
    k_cache: torch.Tensor                # bf16 [1, S, NK, D]
    v_cache: torch.Tensor
    input_norm: torch.Tensor             # fp32 [H]
    post_norm: torch.Tensor
    q_norm: torch.Tensor                 # fp32 [D]
    k_norm: torch.Tensor
    q_weight: torch.Tensor               # uint32 Q4_K words
    k_weight: torch.Tensor
    v_weight: torch.Tensor               # uint32 Q4_K words or uint16 Q6_K halfwords
    o_weight: torch.Tensor
    gate_weight: torch.Tensor
    up_weight: torch.Tensor
    down_weight: torch.Tensor


@dataclass
class ModelTensors:
    decode_layers: list[DecodeLayerTensors]


_MODEL: ModelTensors | None = None


def _physical(w: torch.Tensor, wtype: str) -> torch.Tensor:
    """A packed GGUF row tensor (uint8 [N, row_bytes]) as the reference's word / halfword tensor."""
    return w.view(torch.uint32) if wtype == "q4_k" else w.view(torch.uint16)


def bind_model_tensors(decoder) -> ModelTensors:
    """Build the per-layer tensor sets over a Qwen3Decoder's weights, caches and residual stream, and make them
    the ones run_decode_layer uses (the reference's model_tensors())."""
    global _MODEL
    c = decoder.config
    dev = decoder.device
    hidden = decoder.h.view(1, 1, c.hidden)
    bf, f32 = torch.bfloat16, torch.float32
    normed = torch.zeros(1, 1, c.hidden, dtype=bf, device=dev)
    q = torch.zeros(1, 1, c.q_dim, dtype=f32, device=dev)
    k = torch.zeros(1, 1, c.kv_dim, dtype=f32, device=dev)
    v = torch.zeros(1, 1, c.kv_dim, dtype=f32, device=dev)
    attn = torch.zeros(1, c.heads, 1, c.head_dim, dtype=bf, device=dev)
    gate = torch.zeros(1, 1, c.mlp, dtype=f32, device=dev)
    up = torch.zeros(1, 1, c.mlp, dtype=f32, device=dev)
    act = torch.zeros(1, 1, c.mlp, dtype=bf, device=dev)
    layers = []
    for i in range(c.layers):
        p = f"layers.{i}."
        w = {n: _physical(decoder.weights.packed[p + n], decoder.types[p + n])
             for n in ("q", "k", "v", "o", "gate", "up", "down")}
        layers.append(DecodeLayerTensors(
            hidden=hidden, normed=normed, q=q, k=k, v=v, attn=attn, gate=gate, up=up, act=act,
            k_cache=decoder.k_cache[i].unsqueeze(0), v_cache=decoder.v_cache[i].unsqueeze(0),
            input_norm=decoder.weights.norms[p + "input_norm"], post_norm=decoder.weights.norms[p + "post_norm"],
            q_norm=decoder.weights.norms[p + "q_norm"], k_norm=decoder.weights.norms[p + "k_norm"],
            q_weight=w["q"], k_weight=w["k"], v_weight=w["v"], o_weight=w["o"], gate_weight=w["gate"],
            up_weight=w["up"], down_weight=w["down"]))
    _MODEL = ModelTensors(decode_layers=layers)
    return _MODEL


def model_tensors() -> ModelTensors:
    if _MODEL is None:
        raise RuntimeError("no model tensors bound: call bind_model_tensors(decoder) first")
    return _MODEL


def _linear_q4_or_q6_add(rt: RuntimeSession, *, x: torch.Tensor, weight: torch.Tensor, residual: torch.Tensor,
                         output: torch.Tensor) -> None:
    """decode_layer.py:22-35: the Q6_K variant for halfword weights, else Q4_K."""
    if weight.dtype == torch.uint16:
        V.LINEAR_NOBIAS_Q6_K_MATVEC_ADD_F32(rt, x=x, weight=weight, residual=residual, output=output)
        return
    V.LINEAR_NOBIAS_Q4_K_MATVEC_ADD_F32(rt, x=x, weight=weight, residual=residual, output=output)


def _attn_qkv(rt: RuntimeSession, t: DecodeLayerTensors) -> None:
    """decode_layer.py:38-57."""
    variant = V.LINEAR_NOBIAS_Q4_QK_Q6_V_MATVEC_F32 if t.v_weight.dtype == torch.uint16 \
        else V.LINEAR_NOBIAS_Q4_K_QKV_MATVEC_F32
    variant(rt, x=t.normed, q_weight=t.q_weight, k_weight=t.k_weight, v_weight=t.v_weight, q_output=t.q,
            k_output=t.k, v_output=t.v)


def _run_decode_layer_with_tensors(rt: RuntimeSession, t: DecodeLayerTensors, *, cache_position) -> None:
    nh, d = t.attn.shape[1], t.attn.shape[3]
    nk = t.k_cache.shape[2]
    V.RMS_NORM_MUL_F16_F32(rt, x=t.hidden, weight=t.input_norm, output=t.normed)
    _attn_qkv(rt, t)
    V.SDPA_DECODE_QK_NORM_ROPE_CACHE_WRITE_F32(
        rt, q=t.q.view(1, nh, 1, d), new_k=t.k.view(1, nk, 1, d), new_v=t.v.view(1, 1, nk, d),
        q_norm_weight=t.q_norm, k_norm_weight=t.k_norm, k_cache=t.k_cache, v_cache=t.v_cache,
        cache_position=cache_position, output=t.attn)
    _linear_q4_or_q6_add(rt, x=t.attn.view(1, 1, nh * d), weight=t.o_weight, residual=t.hidden, output=t.hidden)
    V.RMS_NORM_MUL_F16_F32(rt, x=t.hidden, weight=t.post_norm, output=t.normed)
    V.LINEAR_NOBIAS_Q4_K_QK_MATVEC_F32(rt, x=t.normed, q_weight=t.gate_weight, k_weight=t.up_weight,
                                       q_output=t.gate, k_output=t.up)
    V.SWIGLU_F16(rt, gate=t.gate, up=t.up, output=t.act)
    _linear_q4_or_q6_add(rt, x=t.act, weight=t.down_weight, residual=t.hidden, output=t.hidden)


def run_decode_layer(rt: RuntimeSession, layer_idx: int, *, cache_position) -> None:
    """One decoder layer at ``cache_position`` (an int, or a one-element int32 device tensor)
    (src/models/optimized_qwen3/dispatch/decode_layer.py:131-136)."""
    _run_decode_layer_with_tensors(rt, model_tensors().decode_layers[layer_idx], cache_position=cache_position)
