"""CPU oracle of the Qwen3-ASR audio tower (TEST INFRASTRUCTURE ONLY).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import this module.
It is the checker for the HIP path, never the thing measured or shipped.

``audio_tower_cpu`` restates the reference's module semantics (src/models/quantized_qwen3_asr/
pytorch_modules.py:452-526: ``_run_audio_tower``, ``_run_audio_layer``, ``_run_audio_attention``) in fp32
torch on the CPU over weights dequantized from the same Q8_0 bytes the GPU reads.  Its building blocks are
library routines (F.conv2d, F.layer_norm, F.gelu, softmax); what they are pinned by is in
tests/test_asr_host.py: conv2d against the reference shader's index formula on brute-force loops, the
block-diagonal mask against per-window attention, LayerNorm and GELU against their closed forms.
"""

from __future__ import annotations

import math

import numpy as np
import torch
import torch.nn.functional as F

from oracle import quant

PREFIX = "thinker.audio_tower."


def dense_from_packed(packed: dict[str, np.ndarray], vectors: dict[str, np.ndarray],
                      shapes: dict[str, tuple[int, ...]]) -> dict[str, torch.Tensor]:
    """fp32 tensors of the checkpoint shapes from Q8_0 rows (the zero padding of each row dropped)."""
    out = {}
    for name, shape in shapes.items():
        if len(shape) == 1:
            out[name] = torch.from_numpy(np.asarray(vectors[name], np.float32).copy())
            continue
        w = np.asarray(packed[name])
        cols = w.shape[1] // 34 * 32
        k = int(np.prod(shape[1:]))
        deq = quant.dequant_q8_0(w, cols)[:, :k]
        out[name] = torch.from_numpy(np.ascontiguousarray(deq, np.float32)).reshape(shape)
    return out


def conv2d_brute(x: np.ndarray, w: np.ndarray, b: np.ndarray, stride: int, pad: int) -> np.ndarray:
    """Direct loops with the reference shader's addressing: ih = oh*stride + fh - pad, iw = ow*stride + fw - pad,
    taps outside the input skipped (src/models/quantized_qwen3_asr/shaders/conv2d_q8_0w_f32b_f16.py:114-136)."""
    bsz, ci, h, wd = x.shape
    co, _, kh, kw = w.shape
    ho = (h + 2 * pad - kh) // stride + 1
    wo = (wd + 2 * pad - kw) // stride + 1
    y = np.zeros((bsz, co, ho, wo), np.float64)
    for n in range(bsz):
        for oc in range(co):
            for oh in range(ho):
                for ow in range(wo):
                    acc = float(b[oc])
                    for ic in range(ci):
                        for fh in range(kh):
                            for fw in range(kw):
                                ih, iw = oh * stride + fh - pad, ow * stride + fw - pad
                                if 0 <= ih < h and 0 <= iw < wd:
                                    acc += float(x[n, ic, ih, iw]) * float(w[oc, ic, fh, fw])
                    y[n, oc, oh, ow] = acc
    return y


def masked_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, mask: torch.Tensor | None,
                     scale: float) -> torch.Tensor:
    """softmax(q k^T * scale + mask) v over [H, T, D] (scaled_dot_product_attention semantics,
    pytorch_modules.py:511-519)."""
    s = torch.matmul(q, k.transpose(-1, -2).contiguous()) * scale
    if mask is not None:
        s = s + mask
    return torch.matmul(torch.softmax(s, dim=-1), v)


def windowed_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cu_seqlens, scale: float) -> torch.Tensor:
    """The same attention run window by window (no mask): [H, T, D]."""
    out = torch.zeros_like(q)
    cu = [int(c) for c in cu_seqlens]
    for lo, hi in zip(cu[:-1], cu[1:]):
        out[:, lo:hi] = masked_attention(q[:, lo:hi], k[:, lo:hi], v[:, lo:hi], None, scale)
    return out


def gelu(x: torch.Tensor) -> torch.Tensor:
    return F.gelu(x)


def audio_tower_cpu(w: dict[str, torch.Tensor], cfg, padded_feature: np.ndarray, position_embedding: np.ndarray,
                    compact_index: np.ndarray, attention_mask: np.ndarray | None = None,
                    cu_seqlens=None) -> torch.Tensor:
    """fp32 [tokens, output_dim] (``_run_audio_tower``, pytorch_modules.py:452-481).  Attention takes the
    additive mask when given, else runs window by window over ``cu_seqlens``."""
    p = PREFIX
    x = torch.from_numpy(np.asarray(padded_feature, np.float32))
    for n in ("conv2d1", "conv2d2", "conv2d3"):
        x = gelu(F.conv2d(x, w[p + n + ".weight"], w[p + n + ".bias"], stride=2, padding=1))
    b, c, f, t = x.shape
    h = x.reshape(b, c * f, t).transpose(1, 2) @ w[p + "conv_out.weight"].T
    h = h + torch.from_numpy(np.asarray(position_embedding, np.float32))
    h = h.reshape(-1, h.shape[-1])[torch.from_numpy(np.asarray(compact_index, np.int64))]
    mask = None if attention_mask is None else torch.from_numpy(np.asarray(attention_mask, np.float32))[0, 0]
    h = encoder_layers_cpu(w, cfg, h, mask=mask, cu_seqlens=cu_seqlens)
    return encoder_head_cpu(w, cfg, h)


def encoder_layers_cpu(w: dict[str, torch.Tensor], cfg, h: torch.Tensor, *, mask: torch.Tensor | None = None,
                       cu_seqlens=None) -> torch.Tensor:
    """Every pre-LN encoder layer over the fp32 residual stream h [T, d_model] (``_run_audio_layer``,
    pytorch_modules.py:484-526): attention under the additive ``mask`` [T, T] when given, else window by
    window over ``cu_seqlens``."""
    p = PREFIX
    hd = cfg.d_model // cfg.heads
    scale = 1.0 / math.sqrt(hd)
    for i in range(cfg.layers):
        lp = f"{p}layers.{i}."
        res = h
        y = F.layer_norm(h, (cfg.d_model,), w[lp + "self_attn_layer_norm.weight"], w[lp + "self_attn_layer_norm.bias"],
                         eps=cfg.eps)
        seq = y.shape[0]

        def proj(n: str) -> torch.Tensor:
            z = y @ w[lp + f"self_attn.{n}.weight"].T + w[lp + f"self_attn.{n}.bias"]
            return z.reshape(seq, cfg.heads, hd).transpose(0, 1)

        q, k, v = proj("q_proj"), proj("k_proj"), proj("v_proj")
        if mask is not None:
            a = masked_attention(q, k, v, mask, scale)
        else:
            a = windowed_attention(q, k, v, cu_seqlens, scale)
        a = a.transpose(0, 1).reshape(seq, -1)
        h = res + a @ w[lp + "self_attn.out_proj.weight"].T + w[lp + "self_attn.out_proj.bias"]
        res = h
        y = F.layer_norm(h, (cfg.d_model,), w[lp + "final_layer_norm.weight"], w[lp + "final_layer_norm.bias"],
                         eps=cfg.eps)
        y = gelu(y @ w[lp + "fc1.weight"].T + w[lp + "fc1.bias"])
        h = res + y @ w[lp + "fc2.weight"].T + w[lp + "fc2.bias"]
    return h


def encoder_head_cpu(w: dict[str, torch.Tensor], cfg, h: torch.Tensor) -> torch.Tensor:
    """ln_post -> proj1 + GELU -> proj2 (pytorch_modules.py:476-481): fp32 [T, output_dim]."""
    p = PREFIX
    y = F.layer_norm(h, (cfg.d_model,), w[p + "ln_post.weight"], w[p + "ln_post.bias"], eps=cfg.eps)
    y = gelu(y @ w[p + "proj1.weight"].T + w[p + "proj1.bias"])
    return y @ w[p + "proj2.weight"].T + w[p + "proj2.bias"]
