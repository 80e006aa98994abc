"""Audio-tower shapes.

The Qwen3-ASR-0.6B tower (src/models/quantized_qwen3_asr/tensors/audio_encoder.py:129-1305): three 3x3
stride-2 conv2d of 480 channels over 128 mel bins, conv_out 7680 -> 896, 18 pre-LN encoder layers of
14 heads x 64 with a 3584 GELU MLP, ln_post, proj1 (GELU), proj2 896 -> 1024 (the text model's hidden size).
"""

from __future__ import annotations

from dataclasses import dataclass

AUDIO_TOKEN_ID = 151676  # <|audio_pad|>, pytorch_modules.py:116
CONV_KERNEL = 3
CONV_STRIDE = 2
CONV_PAD = 1  # conv2d_q8_0w_f32b_f16.py:67-72


@dataclass(frozen=True)
class AudioEncoderConfig:
    d_model: int
    layers: int
    heads: int
    ffn: int
    output_dim: int
    conv_channels: int = 480
    mel_bins: int = 128
    n_window: int = 50          # a chunk is 2 * n_window mel frames (pytorch_modules.py:54)
    n_window_infer: int = 800   # attention window in mel frames (pytorch_modules.py:90)
    eps: float = 1e-5           # layer_norm_f32w_f32b_f32.py:57

    @property
    def head_dim(self) -> int:
        return self.d_model // self.heads

    @property
    def chunk_frames(self) -> int:
        return 2 * self.n_window

    @property
    def freq_after_conv(self) -> int:
        f = self.mel_bins
        for _ in range(3):
            f = (f + 2 * CONV_PAD - CONV_KERNEL) // CONV_STRIDE + 1
        return f

    @property
    def conv_out_in(self) -> int:
        return self.conv_channels * self.freq_after_conv

    def __post_init__(self) -> None:
        if self.d_model % self.heads or self.head_dim not in (64, 128):
            raise ValueError(f"head_dim {self.d_model}/{self.heads} must be 64 or 128")
        for name in ("d_model", "ffn", "output_dim"):
            if getattr(self, name) % 64:
                raise ValueError(f"{name} must be a multiple of 64 (the GEMM's K step)")


QWEN3_ASR_0_6B_AUDIO = AudioEncoderConfig(d_model=896, layers=18, heads=14, ffn=3584, output_dim=1024)

# the encoder shape of the ASR benchmark configuration: 24 layers, hidden 1024, 16 heads, FFN 4096
ASR_C5_ENCODER = AudioEncoderConfig(d_model=1024, layers=24, heads=16, ffn=4096, output_dim=1024)
