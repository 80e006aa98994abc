"""The Qwen3-ASR audio tower on libt2h.

Op order of the reference's ``run_audio_encoder`` (src/models/quantized_qwen3_asr/dispatch/audio_encoder.py:27-63,
module semantics pytorch_modules.py:452-526), with the MI355X layout:

* conv2d x 3 (3x3, stride 2, pad 1) + GELU: ``t2h_im2col`` patch rows, then one Q8_0 GEMM with the bias and
  the GELU in its epilogue.  Activations stay channels-last [chunk, h, w, 480] bf16, so each im2col reads
  consecutive channels;
* conv_out (no bias) over the (channel, frequency) rows of every time step, with the sinusoidal position
  table added in the GEMM epilogue (fp32 out), then the valid tokens gathered (``index_select``);
* per layer: LayerNorm -> one Q8_0 GEMM for q|k|v (stacked rows, stacked biases) -> attention within the
  windows (``t2h_flash_attn_segments``: no [T, T] mask is built or read) -> out_proj with the residual added in
  its epilogue -> LayerNorm -> fc1 + bias + GELU -> fc2 + bias + residual.  The residual stream is fp32; GEMM
  inputs are bf16;
* ln_post -> proj1 + GELU -> proj2 (fp32 [T, output_dim]).

Every tensor the kernels read is allocated by the caller's PyTorch caching allocator; nothing runs on the CPU.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import torch

from torch2vk_amd import kernels
from torch2vk_amd.qwen3_asr.config import CONV_KERNEL, CONV_PAD, CONV_STRIDE, AudioEncoderConfig

PREFIX = "thinker.audio_tower."


def audio_tensor_shapes(cfg: AudioEncoderConfig) -> dict[str, tuple[int, ...]]:
    """Checkpoint names and shapes of the tower (src/models/quantized_qwen3_asr/tensors/audio_encoder.py)."""
    d, f, c = cfg.d_model, cfg.ffn, cfg.conv_channels
    shapes: dict[str, tuple[int, ...]] = {
        "conv2d1.weight": (c, 1, CONV_KERNEL, CONV_KERNEL), "conv2d1.bias": (c,),
        "conv2d2.weight": (c, c, CONV_KERNEL, CONV_KERNEL), "conv2d2.bias": (c,),
        "conv2d3.weight": (c, c, CONV_KERNEL, CONV_KERNEL), "conv2d3.bias": (c,),
        "conv_out.weight": (d, cfg.conv_out_in),
        "ln_post.weight": (d,), "ln_post.bias": (d,),
        "proj1.weight": (d, d), "proj1.bias": (d,),
        "proj2.weight": (cfg.output_dim, d), "proj2.bias": (cfg.output_dim,),
    }
    for i in range(cfg.layers):
        p = f"layers.{i}."
        for n in ("q_proj", "k_proj", "v_proj", "out_proj"):
            shapes[p + f"self_attn.{n}.weight"] = (d, d)
            shapes[p + f"self_attn.{n}.bias"] = (d,)
        for n in ("self_attn_layer_norm", "final_layer_norm"):
            shapes[p + f"{n}.weight"] = (d,)
            shapes[p + f"{n}.bias"] = (d,)
        shapes[p + "fc1.weight"] = (f, d)
        shapes[p + "fc1.bias"] = (f,)
        shapes[p + "fc2.weight"] = (d, f)
        shapes[p + "fc2.bias"] = (d,)
    return {PREFIX + k: v for k, v in shapes.items()}


def q8_0_cols(shape: tuple[int, ...]) -> int:
    """Row length of a Q8_0 matrix: the product of the trailing dims, padded to a whole 32-value block
    (src/torch2vk/quantize/gguf.py:119-124,311-315)."""
    k = 1
    for s in shape[1:]:
        k *= s
    return -(-k // 32) * 32


@dataclass
class AudioEncoderWeights:
    """Q8_0 rows (uint8 [N, 34 * blocks]) for every matrix and conv kernel, fp32 vectors for biases and norms,
    under the checkpoint names.  ``qkv`` holds each layer's q|k|v rows stacked in one allocation."""

    config: AudioEncoderConfig
    packed: dict[str, torch.Tensor]
    vectors: dict[str, torch.Tensor]
    qkv: list[tuple[torch.Tensor, torch.Tensor]] = field(default_factory=list)

    def stack_qkv(self) -> None:
        self.qkv = []
        for i in range(self.config.layers):
            p = f"{PREFIX}layers.{i}.self_attn."
            w = torch.cat([self.packed[p + f"{n}.weight"] for n in ("q_proj", "k_proj", "v_proj")], dim=0)
            b = torch.cat([self.vectors[p + f"{n}.bias"] for n in ("q_proj", "k_proj", "v_proj")], dim=0)
            self.qkv.append((w.contiguous(), b.contiguous()))

    def packed_bytes(self) -> int:
        return sum(t.numel() for t in self.packed.values())


def quantize_audio_weights(dense: dict[str, torch.Tensor], cfg: AudioEncoderConfig, device) -> AudioEncoderWeights:
    """Checkpoint tensors (fp32, any device) -> Q8_0 rows through the GPU quantizer (bit-identical to the
    reference's GGUF_QUANTIZE_Q8_0_F32, src/torch2vk/quantize/vulkan.py:91-185); every tensor of two or more
    dims is Q8_0, as the reference's Qwen3-ASR policy forces for the audio tower
    (src/models/quantized_qwen3_asr/quantization.py:8-9)."""
    packed, vectors = {}, {}
    for name, shape in audio_tensor_shapes(cfg).items():
        t = dense[name].to(device=device, dtype=torch.float32)
        if tuple(t.shape) != shape:
            raise ValueError(f"{name}: shape {tuple(t.shape)}, expected {shape}")
        if len(shape) == 1:
            vectors[name] = t.contiguous()
            continue
        rows, cols = shape[0], q8_0_cols(shape)
        flat = t.reshape(rows, -1)
        if flat.shape[1] != cols:
            flat = torch.nn.functional.pad(flat, (0, cols - flat.shape[1]))
        packed[name] = kernels.quantize(flat.contiguous(), "q8_0")
    w = AudioEncoderWeights(cfg, packed, vectors)
    w.stack_qkv()
    return w


def synthetic_audio_dense(cfg: AudioEncoderConfig, *, seed: int = 0, std: float = 0.02) -> dict[str, torch.Tensor]:
    """Random-init fp32 checkpoint on the CPU: matrices and conv kernels ~N(0, std) (conv kernels scaled by
    1/sqrt(fan_in) / 0.02 * std so that activations stay O(1)), biases ~N(0, std), LayerNorm weights
    1 + N(0, std), LayerNorm biases N(0, std).  Drawn in the order of ``audio_tensor_shapes``."""
    g = torch.Generator("cpu").manual_seed(seed)
    out = {}
    for name, shape in audio_tensor_shapes(cfg).items():
        t = torch.randn(shape, generator=g, dtype=torch.float32) * std
        if name.endswith("norm.weight") or name.endswith("ln_post.weight"):
            t = t + 1.0
        elif len(shape) == 4:
            fan_in = shape[1] * shape[2] * shape[3]
            t = t * (1.0 / (fan_in ** 0.5) / 0.02)
        out[name] = t
    return out


class Qwen3AudioEncoder:
    """The audio tower over libt2h kernels (run_audio_encoder, dispatch/audio_encoder.py:27-63)."""

    def __init__(self, weights: AudioEncoderWeights) -> None:
        self.weights = weights
        self.config = weights.config
        if not weights.qkv:
            weights.stack_qkv()

    def _p(self, name: str) -> torch.Tensor:
        return self.weights.packed[PREFIX + name]

    def _v(self, name: str) -> torch.Tensor:
        return self.weights.vectors[PREFIX + name]

    # ------------------------------------------------------- front-end --

    def _conv(self, x_nchw: torch.Tensor, name: str) -> torch.Tensor:
        """conv2d (3x3, stride 2, pad 1) + bias + GELU; x [B, C, H, W] view -> channels-last bf16 [B, Ho, Wo, Co]."""
        b, _, h, w = x_nchw.shape
        ho = kernels.conv_out_size(h, CONV_KERNEL, CONV_STRIDE, CONV_PAD)
        wo = kernels.conv_out_size(w, CONV_KERNEL, CONV_STRIDE, CONV_PAD)
        cols = kernels.im2col(x_nchw, (CONV_KERNEL, CONV_KERNEL), (CONV_STRIDE, CONV_STRIDE), (CONV_PAD, CONV_PAD))
        y = kernels.q8_0_linear(cols, self._p(name + ".weight"), bias=self._v(name + ".bias"), act="gelu")
        return y.view(b, ho, wo, -1)

    def frontend(self, padded_feature: torch.Tensor, position_embedding: torch.Tensor) -> torch.Tensor:
        """[chunks, 1, mel, frames] fp32 -> fp32 [chunks * tokens, d_model] = conv_out(...) + position table."""
        cfg = self.config
        x = padded_feature
        y = self._conv(x, "conv2d1")
        y = self._conv(y.permute(0, 3, 1, 2), "conv2d2")
        y = self._conv(y.permute(0, 3, 1, 2), "conv2d3")
        chunks, f, t, _ = y.shape
        # rows (chunk, time), columns (channel, frequency): an (f x 1) patch over each time step
        rows = kernels.im2col(y.permute(0, 3, 1, 2), (f, 1))
        pos = position_embedding.reshape(chunks * t, cfg.d_model)
        return kernels.q8_0_linear(rows, self._p("conv_out.weight"), out_dtype=torch.float32, residual=pos)

    # --------------------------------------------------------- encoder --

    def encoder_layer(self, i: int, h: torch.Tensor, cu: torch.Tensor) -> None:
        """One pre-LN layer on the fp32 residual stream h [T, d_model], in place (pytorch_modules.py:484-526)."""
        cfg = self.config
        p = f"layers.{i}."
        t_len, d = h.shape
        x = kernels.layer_norm(h, self._v(p + "self_attn_layer_norm.weight"), self._v(p + "self_attn_layer_norm.bias"),
                               eps=cfg.eps)
        w_qkv, b_qkv = self.weights.qkv[i]
        qkv = kernels.q8_0_linear(x, w_qkv, bias=b_qkv)
        hd = cfg.head_dim
        q = qkv[:, :d].view(1, t_len, cfg.heads, hd)
        k = qkv[:, d:2 * d].view(1, t_len, cfg.heads, hd)
        v = qkv[:, 2 * d:].view(1, t_len, cfg.heads, hd)
        attn = kernels.flash_attn_segments(q, k, v, cu)
        kernels.q8_0_linear(attn.view(t_len, d), self._p(p + "self_attn.out_proj.weight"),
                            bias=self._v(p + "self_attn.out_proj.bias"), out=h, residual=h)
        x = kernels.layer_norm(h, self._v(p + "final_layer_norm.weight"), self._v(p + "final_layer_norm.bias"),
                               eps=cfg.eps)
        f1 = kernels.q8_0_linear(x, self._p(p + "fc1.weight"), bias=self._v(p + "fc1.bias"), act="gelu")
        kernels.q8_0_linear(f1, self._p(p + "fc2.weight"), bias=self._v(p + "fc2.bias"), out=h, residual=h)

    def encoder_layers(self, h: torch.Tensor, cu_seqlens) -> torch.Tensor:
        cu = kernels.segment_bounds(cu_seqlens, int(h.shape[0]), h.device)
        for i in range(self.config.layers):
            self.encoder_layer(i, h, cu)
        return h

    def head(self, h: torch.Tensor) -> torch.Tensor:
        """ln_post -> proj1 + GELU -> proj2: fp32 [T, output_dim]."""
        x = kernels.layer_norm(h, self._v("ln_post.weight"), self._v("ln_post.bias"), eps=self.config.eps)
        x = kernels.q8_0_linear(x, self._p("proj1.weight"), bias=self._v("proj1.bias"), act="gelu")
        return kernels.q8_0_linear(x, self._p("proj2.weight"), bias=self._v("proj2.bias"), out_dtype=torch.float32)

    def run_audio_encoder(self, padded_feature: torch.Tensor, position_embedding: torch.Tensor,
                          compact_index: torch.Tensor, cu_seqlens) -> torch.Tensor:
        """Preprocessed inputs (``preprocess.preprocess_audio_inputs``) on the device -> audio features
        fp32 [tokens, output_dim]."""
        grid = self.frontend(padded_feature, position_embedding)
        h = kernels.index_select_rows(grid, compact_index)
        self.encoder_layers(h, cu_seqlens)
        return self.head(h)


def run_audio_inject(inputs_embeds: torch.Tensor, audio_positions: torch.Tensor,
                     audio_features: torch.Tensor) -> torch.Tensor:
    """inputs_embeds[audio_positions[i]] = audio_features[i], in place (run_audio_inject,
    dispatch/audio_inject.py:11-13; torch.index_copy along the token axis, pytorch_modules.py:16-28)."""
    emb = inputs_embeds.reshape(-1, inputs_embeds.shape[-1])
    return kernels.index_copy_rows(emb, audio_positions, audio_features.reshape(-1, emb.shape[-1]))
