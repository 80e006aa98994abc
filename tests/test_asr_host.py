"""Qwen3-ASR host logic and the audio-tower oracle, on the CPU.

The preprocessing (chunking, token counts, windows, position table) is pinned against closed forms and
brute force; the oracle's building blocks against the reference shader's conv indexing, per-window attention,
and the closed forms of LayerNorm and GELU."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import asr as oasr
from oracle import quant
from torch2vk_amd.qwen3_asr import config as acfg
from torch2vk_amd.qwen3_asr import preprocess as pp
from torch2vk_amd.qwen3_asr.encoder import audio_tensor_shapes, q8_0_cols, synthetic_audio_dense

TINY = acfg.AudioEncoderConfig(d_model=128, layers=2, heads=2, ffn=256, output_dim=128, conv_channels=32)


def _conv_len(n: int) -> int:
    return (n + 2 * acfg.CONV_PAD - acfg.CONV_KERNEL) // acfg.CONV_STRIDE + 1


def test_feat_extract_output_lengths_is_three_convs_per_chunk():
    for total in range(1, 651):
        brute = 0
        left = total
        while left > 0:
            n = min(left, 100)
            brute += _conv_len(_conv_len(_conv_len(n)))
            left -= n
        assert int(pp.feat_extract_output_lengths(total)) == brute, total
    assert int(pp.feat_extract_output_lengths(100)) == 13
    assert pp.tokens_per_chunk(acfg.QWEN3_ASR_0_6B_AUDIO) == 13


def test_sinusoid_position_embedding_closed_form():
    length, channels = 13, 896
    pe = pp.sinusoid_position_embedding(length, channels)
    assert pe.shape == (length, channels) and pe.dtype == np.float32
    half = channels // 2
    np.testing.assert_array_equal(pe[0, :half], 0.0)
    np.testing.assert_array_equal(pe[0, half:], 1.0)
    for t, i in ((1, 0), (5, 7), (12, 300), (12, half - 1)):
        ang = t * 10000.0 ** (-i / (half - 1))
        assert abs(pe[t, i] - math.sin(ang)) < 1e-6
        assert abs(pe[t, half + i] - math.cos(ang)) < 1e-6


def test_windows_and_block_diagonal_mask():
    cu = pp.window_bounds(250, 104)
    np.testing.assert_array_equal(cu, [0, 104, 208, 250])
    assert pp.window_bounds(104, 104).tolist() == [0, 104]
    mask = pp.block_diagonal_mask(cu)[0, 0]
    win = np.searchsorted(cu, np.arange(250), side="right") - 1
    same = win[:, None] == win[None, :]
    assert (mask[same] == 0).all()
    assert (mask[~same] == np.finfo(np.float32).min).all()


def test_preprocess_one_utterance():
    rng = np.random.default_rng(0)
    frames = 1234
    mel = rng.standard_normal((1, 128, frames + 30)).astype(np.float32)
    ids = np.array([1, 2, acfg.AUDIO_TOKEN_ID, acfg.AUDIO_TOKEN_ID, 5, acfg.AUDIO_TOKEN_ID])
    fmask = np.zeros((1, frames + 30), np.int64)
    fmask[0, :frames] = 1
    cfg = acfg.QWEN3_ASR_0_6B_AUDIO
    out = pp.preprocess_audio_inputs(ids, mel, fmask, cfg, with_mask=True)
    padded = out["padded_feature"]
    assert padded.shape == (13, 1, 128, 100)
    flat = np.concatenate([padded[i, 0] for i in range(13)], axis=1)
    np.testing.assert_array_equal(flat[:, :frames], mel[0, :, :frames])
    assert (flat[:, frames:] == 0).all()
    n_tok = int(pp.feat_extract_output_lengths(frames))
    ci = out["compact_index"]
    assert ci.dtype == np.int64 and ci.size == n_tok
    expected = np.concatenate([i * 13 + np.arange(13) for i in range(12)] + [12 * 13 + np.arange(_conv_len(
        _conv_len(_conv_len(34))))])
    np.testing.assert_array_equal(ci, expected)
    assert out["cu_seqlens"].tolist() == [0, 104, n_tok]
    assert out["position_embedding"].shape == (13, 13, 896)
    np.testing.assert_array_equal(out["position_embedding"][5], pp.sinusoid_position_embedding(13, 896))
    np.testing.assert_array_equal(out["audio_positions"], [2, 3, 5])
    assert out["audio_attention_mask"].shape == (1, 1, n_tok, n_tok)


def test_audio_tower_shapes_of_qwen3_asr_0_6b():
    cfg = acfg.QWEN3_ASR_0_6B_AUDIO
    shapes = audio_tensor_shapes(cfg)
    p = "thinker.audio_tower."
    assert cfg.freq_after_conv == 16 and cfg.head_dim == 64
    assert shapes[p + "conv2d1.weight"] == (480, 1, 3, 3)
    assert shapes[p + "conv2d2.weight"] == (480, 480, 3, 3)
    assert shapes[p + "conv_out.weight"] == (896, 7680)
    assert shapes[p + "layers.17.fc1.weight"] == (3584, 896)
    assert shapes[p + "proj2.weight"] == (1024, 896)
    assert p + "layers.18.fc1.weight" not in shapes
    assert q8_0_cols(shapes[p + "conv2d1.weight"]) == 32
    assert q8_0_cols(shapes[p + "conv2d2.weight"]) == 4320


def test_conv2d_oracle_follows_the_shader_indexing():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((2, 3, 7, 9)).astype(np.float32)
    w = rng.standard_normal((4, 3, 3, 3)).astype(np.float32)
    b = rng.standard_normal(4).astype(np.float32)
    ref = oasr.conv2d_brute(x, w, b, stride=2, pad=1)
    got = F.conv2d(torch.from_numpy(x), torch.from_numpy(w), torch.from_numpy(b), stride=2, padding=1).numpy()
    np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-5)


def test_block_diagonal_mask_equals_windowed_attention():
    g = torch.Generator().manual_seed(2)
    q, k, v = (torch.randn(3, 50, 16, generator=g) for _ in range(3))
    cu = [0, 13, 30, 50]
    mask = torch.from_numpy(pp.block_diagonal_mask(np.array(cu))[0, 0])
    a = oasr.masked_attention(q, k, v, mask, 0.25)
    b = oasr.windowed_attention(q, k, v, cu, 0.25)
    torch.testing.assert_close(a, b, rtol=1e-6, atol=1e-6)


def test_layer_norm_and_gelu_closed_forms():
    g = torch.Generator().manual_seed(3)
    x = torch.randn(5, 64, generator=g, dtype=torch.float64) * 3 + 1
    w, b = torch.randn(64, generator=g, dtype=torch.float64), torch.randn(64, generator=g, dtype=torch.float64)
    mean = x.mean(-1, keepdim=True)
    var = ((x - mean) ** 2).mean(-1, keepdim=True)
    torch.testing.assert_close(F.layer_norm(x, (64,), w, b, eps=1e-5), (x - mean) / torch.sqrt(var + 1e-5) * w + b)
    xs = np.linspace(-6, 6, 241)
    exact = np.array([0.5 * t * (1 + math.erf(t / math.sqrt(2))) for t in xs])
    np.testing.assert_allclose(F.gelu(torch.from_numpy(xs)).numpy(), exact, rtol=0, atol=1e-12)


def test_reference_erf_approximation_is_within_its_published_bound():
    """The reference's GELU evaluates erf by Abramowitz-Stegun 7.1.26 (gelu_f32.py:61-73), and so does the build
    (gelu_as in csrc/common.h): the published constants are within 1.5e-7 of the exact erf."""
    p, a = 0.3275911, (0.254829592, -0.284496736, 1.421413741, -1.453152027, 1.061405429)
    for t in np.linspace(-8, 8, 4001):
        u = 1.0 / (1.0 + p * abs(t))
        poly = ((((a[4] * u + a[3]) * u + a[2]) * u + a[1]) * u + a[0]) * u
        approx = math.copysign(1.0 - poly * math.exp(-t * t), t)
        assert abs(approx - math.erf(t)) <= 1.5e-7


def test_oracle_tower_mask_and_windows_agree():
    dense = synthetic_audio_dense(TINY, seed=4)
    rng = np.random.default_rng(4)
    mel = rng.standard_normal((1, 128, 260)).astype(np.float32)
    inp = pp.preprocess_audio_inputs(np.zeros(0), mel, np.ones((1, 260)), TINY, with_mask=True)
    a = oasr.audio_tower_cpu(dense, TINY, inp["padded_feature"], inp["position_embedding"], inp["compact_index"],
                             attention_mask=inp["audio_attention_mask"])
    b = oasr.audio_tower_cpu(dense, TINY, inp["padded_feature"], inp["position_embedding"], inp["compact_index"],
                             cu_seqlens=inp["cu_seqlens"])
    assert a.shape == (int(pp.feat_extract_output_lengths(260)), TINY.output_dim)
    torch.testing.assert_close(a, b, rtol=1e-4, atol=1e-4)


def test_dense_from_packed_round_trips_conv_kernels():
    rng = np.random.default_rng(5)
    w = rng.standard_normal((6, 1, 3, 3)).astype(np.float32)
    flat = np.zeros((6, 32), np.float32)
    flat[:, :9] = w.reshape(6, 9)
    packed = quant.quantize_q8_0(flat)
    dense = oasr.dense_from_packed({"c": packed}, {}, {"c": (6, 1, 3, 3)})["c"].numpy()
    assert dense.shape == (6, 1, 3, 3)
    amax = np.abs(w.reshape(6, 9)).max(axis=1)
    assert (np.abs(dense.reshape(6, 9) - w.reshape(6, 9)) <= amax[:, None] / 127 * 0.5 + 1e-3 * amax[:, None]).all()


@pytest.mark.parametrize("frames", [1, 99, 100, 101, 850])
def test_token_count_matches_windows(frames):
    cfg = acfg.QWEN3_ASR_0_6B_AUDIO
    out = pp.preprocess_audio_inputs(np.zeros(0), np.zeros((128, frames), np.float32), np.ones(frames), cfg)
    n = int(pp.feat_extract_output_lengths(frames))
    assert out["compact_index"].size == n and int(out["cu_seqlens"][-1]) == n
