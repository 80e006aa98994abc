"""OmniVoice's acoustic decoder (run_audio_decode, src/models/quantized_omnivoice/dispatch/audio_decode.py:
60-760) on this library's kernels, activations channels-last [T, C] throughout:

    per codebook c: EMBEDDING_Q8_0 -> LINEAR_BIAS (project_out), summed      (lines 66-141)
    LINEAR_BIAS fc2                                                          (line 145)
    CONV1D conv1 (k 7, pad 3)                                                (line 149)
    per block (stride s): snake -> CONV_TRANSPOSE1D (k 2s, pad ceil(s/2), s outputs per input)
                          -> 3 residual units (dilation 1, 3, 9):
                             x + conv_k1(snake(conv_k7,dil(snake(x))))       (lines 151-740)
    snake -> CONV1D conv2 (k 7, pad 3, one output channel)                   (lines 741-755)

Q8_0 weights are the reference's rows as stored: [out, in * k] for conv1d and linears, [in, out * k] for
conv_transpose1d (each row padded to whole 32-value blocks).
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np
import torch

from torch2vk_amd import kernels

DILATIONS = (1, 3, 9)


@dataclass(frozen=True)
class AudioDecoderConfig:
    codebooks: int
    vocab: int
    codebook_dim: int
    latent: int
    hidden: int
    channels: int              # conv1's output channels; each block halves them
    strides: tuple[int, ...]


def out_len(cfg: AudioDecoderConfig, t: int) -> int:
    """Waveform samples for t codec frames: each block's transposed conv (kernel 2s, padding ceil(s/2), output
    padding s % 2) writes s outputs per input, as the reference's tensors are sized (target_len * 8, * 40, * 160,
    * 320, * 960 for strides 8, 5, 4, 2, 3: src/models/quantized_omnivoice/tensors/audio_decode.py)."""
    for s in cfg.strides:
        t = (t - 1) * s - 2 * math.ceil(s / 2) + 2 * s + s % 2
    return t


def dense_shapes(cfg: AudioDecoderConfig) -> dict[str, tuple[int, ...]]:
    """Logical fp32 shapes: matrices as the rows the reference quantizes, vectors [n]."""
    s = {}
    for c in range(cfg.codebooks):
        s[f"cb{c}"] = (cfg.vocab, cfg.codebook_dim)
        s[f"proj{c}.w"] = (cfg.latent, cfg.codebook_dim)
        s[f"proj{c}.b"] = (cfg.latent,)
    s["fc2.w"], s["fc2.b"] = (cfg.hidden, cfg.latent), (cfg.hidden,)
    s["conv1.w"], s["conv1.b"] = (cfg.channels, cfg.hidden * 7), (cfg.channels,)
    ch = cfg.channels
    for i, st in enumerate(cfg.strides):
        co = ch // 2
        s[f"b{i}.alpha"] = (ch,)
        s[f"b{i}.convt.w"], s[f"b{i}.convt.b"] = (ch, co * 2 * st), (co,)
        for j in range(len(DILATIONS)):
            p = f"b{i}.r{j}."
            s[p + "a1"], s[p + "a2"] = (co,), (co,)
            s[p + "c1.w"], s[p + "c1.b"] = (co, co * 7), (co,)
            s[p + "c2.w"], s[p + "c2.b"] = (co, co), (co,)
        ch = co
    s["final.alpha"] = (ch,)
    s["conv2.w"], s["conv2.b"] = (1, ch * 7), (1,)
    return s


def synthetic_dense(cfg: AudioDecoderConfig, seed: int = 0) -> dict[str, np.ndarray]:
    rng = np.random.default_rng(seed)
    out = {}
    for name, shape in dense_shapes(cfg).items():
        if "alpha" in name or name.endswith(".a1") or name.endswith(".a2"):
            out[name] = (np.abs(rng.standard_normal(shape)) + 0.3).astype(np.float32)
        elif len(shape) == 1:
            out[name] = (rng.standard_normal(shape) * 0.05).astype(np.float32)
        else:
            fan_in = shape[1] if not name.endswith("convt.w") else shape[0]
            out[name] = (rng.standard_normal(shape) / math.sqrt(fan_in)).astype(np.float32)
    return out


def quantize_rows(w: np.ndarray, device) -> torch.Tensor:
    """Q8_0 rows of w [R, K], zero-padded to whole 32-value blocks as the reference stores them."""
    r, k = w.shape
    kp = (k + 31) // 32 * 32
    full = np.zeros((r, kp), np.float32)
    full[:, :k] = w
    return kernels.quantize(torch.from_numpy(full).to(device), "q8_0")


class OmniVoiceAudioDecoder:
    def __init__(self, cfg: AudioDecoderConfig, dense: dict[str, np.ndarray], device) -> None:
        self.cfg = cfg
        self.device = torch.device(device)
        self.w = {n: (quantize_rows(a, self.device) if a.ndim == 2 else torch.from_numpy(a).to(self.device))
                  for n, a in dense.items()}

    def _unit(self, x: torch.Tensor, p: str, dil: int) -> torch.Tensor:
        w = self.w
        r = kernels.snake(x, w[p + "a1"])
        r = kernels.conv1d_q8_0(r, w[p + "c1.w"], w[p + "c1.b"], 7, padding=3 * dil, dilation=dil)
        r = kernels.snake(r, w[p + "a2"])
        return kernels.conv1d_q8_0(r, w[p + "c2.w"], w[p + "c2.b"], 1, residual=x)

    def decode(self, codes: torch.Tensor, stages: list | None = None) -> torch.Tensor:
        """codes int64 [C, T] -> waveform fp32 [out_len(T)].  ``stages``: a list that receives the fp32
        channels-last activation [T, C] after conv1, after each block's transposed conv and after each of its
        residual units."""
        cfg, w = self.cfg, self.w
        codes = codes.to(device=self.device, dtype=torch.int64)
        t = int(codes.shape[1])
        acc = torch.zeros(t, cfg.latent, dtype=torch.float32, device=self.device)
        for c in range(cfg.codebooks):
            e = kernels.embedding_q8_0(w[f"cb{c}"], codes[c].contiguous(), cfg.codebook_dim)
            cols = kernels.im2col_1d(e.view(1, t, -1), 1)
            kernels.q8_0_linear(cols, w[f"proj{c}.w"], bias=w[f"proj{c}.b"], out=acc, out_dtype=torch.float32,
                                residual=acc)
        h = kernels.q8_0_linear(kernels.im2col_1d(acc.view(1, t, -1), 1), w["fc2.w"], bias=w["fc2.b"],
                                out_dtype=torch.float32)
        x = kernels.conv1d_q8_0(h.view(1, t, -1), w["conv1.w"], w["conv1.b"], 7, padding=3)
        if stages is not None:
            stages.append(x)
        ch = cfg.channels
        for i, s in enumerate(cfg.strides):
            x = kernels.snake(x, w[f"b{i}.alpha"])
            x = kernels.conv_transpose1d_q8_0(x, w[f"b{i}.convt.w"], w[f"b{i}.convt.b"], ch // 2, 2 * s, stride=s,
                                              padding=math.ceil(s / 2), output_padding=s % 2)
            if stages is not None:
                stages.append(x)
            for j, d in enumerate(DILATIONS):
                x = self._unit(x, f"b{i}.r{j}.", d)
                if stages is not None:
                    stages.append(x)
            ch //= 2
        x = kernels.snake(x, w["final.alpha"])
        return kernels.conv1d_q8_0(x, w["conv2.w"], w["conv2.b"], 7, padding=3).view(-1)
