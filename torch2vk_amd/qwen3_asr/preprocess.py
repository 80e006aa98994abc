"""Host-side preparation of one utterance for the audio tower (numpy; nothing here touches the GPU).

Same outputs and meaning as the reference's ``preprocess_audio_inputs``
(src/models/quantized_qwen3_asr/pytorch_modules.py:31-127):

* the mel spectrogram [mel, frames] is cut into chunks of 2 * n_window frames, each zero-padded to full
  length: ``padded_feature`` [chunks, 1, mel, 2 * n_window];
* a chunk of L frames yields ``feat_extract_output_lengths(L)`` tokens after the three stride-2 convs; the
  valid tokens of every chunk, in order, are ``compact_index`` into the [chunks * tokens_per_chunk] grid;
* the encoder attends within windows of ``n_window_infer / (2 n_window)`` chunks' worth of tokens:
  ``cu_seqlens`` are the window bounds, and ``attention_mask`` the equivalent additive block-diagonal mask;
* ``position_embedding`` is the sinusoidal table of one chunk's tokens, repeated for every chunk;
* ``audio_positions`` are the prompt positions holding the audio placeholder token.
"""

from __future__ import annotations

import numpy as np

from torch2vk_amd.qwen3_asr.config import AUDIO_TOKEN_ID, AudioEncoderConfig


def feat_extract_output_lengths(input_lengths) -> np.ndarray:
    """Tokens left after the conv front-end for mel lengths L: 13 per whole 100-frame chunk, and the
    remainder r through three (x - 1) // 2 + 1 halvings (pytorch_modules.py:31-34)."""
    n = np.asarray(input_lengths, dtype=np.int64)
    rem = n % 100
    t = (rem - 1) // 2 + 1
    t = (t - 1) // 2 + 1
    t = (t - 1) // 2 + 1
    return t + (n // 100) * 13


def sinusoid_position_embedding(length: int, channels: int) -> np.ndarray:
    """[length, channels] fp32: sin over the first half, cos over the second, timescales
    10000^(-i / (channels/2 - 1)) (pytorch_modules.py:37-42, evaluated in float64 then rounded once)."""
    half = channels // 2
    inv = np.exp(-np.log(10000.0) / (half - 1) * np.arange(half, dtype=np.float64))
    t = np.arange(length, dtype=np.float64)[:, None] * inv[None, :]
    return np.concatenate([np.sin(t), np.cos(t)], axis=1).astype(np.float32)


def chunk_lengths(feat_len: int, cfg: AudioEncoderConfig) -> np.ndarray:
    full = cfg.chunk_frames
    n = -(-feat_len // full)
    lengths = np.full(n, full, dtype=np.int64)
    if feat_len % full:
        lengths[-1] = feat_len % full
    return lengths


def tokens_per_chunk(cfg: AudioEncoderConfig) -> int:
    return int(feat_extract_output_lengths(cfg.chunk_frames))


def window_bounds(n_tokens: int, window: int) -> np.ndarray:
    """int32 [n_windows + 1]: whole windows of ``window`` tokens, then the remainder (pytorch_modules.py:88-99)."""
    sizes = [window] * (n_tokens // window)
    if n_tokens % window:
        sizes.append(n_tokens % window)
    return np.cumsum([0, *sizes]).astype(np.int32)


def block_diagonal_mask(cu_seqlens: np.ndarray) -> np.ndarray:
    """Additive fp32 [1, 1, T, T] mask: 0 within a window, the lowest finite fp32 elsewhere
    (pytorch_modules.py:101-110)."""
    t = int(cu_seqlens[-1])
    mask = np.full((1, 1, t, t), np.finfo(np.float32).min, dtype=np.float32)
    for lo, hi in zip(cu_seqlens[:-1], cu_seqlens[1:]):
        mask[0, 0, lo:hi, lo:hi] = 0.0
    return mask


def preprocess_audio_inputs(input_ids, input_features, feature_attention_mask, cfg: AudioEncoderConfig, *,
                            with_mask: bool = False) -> dict[str, np.ndarray]:
    """Encoder inputs for one utterance.  input_features [1, mel, frames] (or [mel, frames]); the first
    sum(feature_attention_mask) frames are used."""
    feats = np.asarray(input_features, dtype=np.float32)
    if feats.ndim == 3:
        feats = feats[0]
    feat_len = int(np.asarray(feature_attention_mask).reshape(-1).sum())
    mel = feats[:, :feat_len]
    lengths = chunk_lengths(feat_len, cfg)
    padded = np.zeros((len(lengths), 1, mel.shape[0], cfg.chunk_frames), dtype=np.float32)
    start = 0
    for i, n in enumerate(lengths):
        padded[i, 0, :, :n] = mel[:, start:start + n]
        start += int(n)

    per_chunk = tokens_per_chunk(cfg)
    pos = sinusoid_position_embedding(per_chunk, cfg.d_model)
    position_embedding = np.ascontiguousarray(np.broadcast_to(pos, (len(lengths), per_chunk, cfg.d_model)))

    valid = feat_extract_output_lengths(lengths)
    compact_index = np.concatenate([i * per_chunk + np.arange(int(v)) for i, v in enumerate(valid)]).astype(np.int64)

    window = int(valid.max()) * (cfg.n_window_infer // cfg.chunk_frames)
    n_tokens = int(feat_extract_output_lengths(feat_len))
    cu_seqlens = window_bounds(n_tokens, window)

    out = {
        "padded_feature": padded,
        "position_embedding": position_embedding,
        "compact_index": compact_index,
        "cu_seqlens": cu_seqlens,
        "audio_positions": np.flatnonzero(np.asarray(input_ids).reshape(-1) == AUDIO_TOKEN_ID).astype(np.int64),
    }
    if with_mask:
        out["audio_attention_mask"] = block_diagonal_mask(cu_seqlens)
    return out
