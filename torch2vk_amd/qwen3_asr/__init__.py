"""Qwen3-ASR on libt2h: the audio tower (conv2d front-end + Transformer encoder) and the injection of its
features into the Qwen3 text decoder's prompt embeddings."""

from torch2vk_amd.qwen3_asr.config import ASR_C5_ENCODER, QWEN3_ASR_0_6B_AUDIO, AudioEncoderConfig  # noqa: F401
