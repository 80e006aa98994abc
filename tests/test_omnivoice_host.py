"""CPU pins of the OmniVoice decoder oracle (oracle/omnivoice.py): conv1d against torch's conv1d at the
decoder's kernel sizes, strides, paddings and dilations; snake by its fixed points and period."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import omnivoice as O


@pytest.mark.parametrize("k,stride,pad,dil", [(7, 1, 3, 1), (7, 1, 9, 3), (7, 1, 27, 9), (1, 1, 0, 1), (3, 2, 1, 1),
                                              (4, 3, 0, 2), (7, 1, 0, 1)])
def test_conv1d_ref_matches_torch(k, stride, pad, dil):
    rng = np.random.default_rng(k * 100 + dil)
    b, c, co, length = 2, 5, 6, 40
    x = rng.standard_normal((b, c, length))
    w = rng.standard_normal((co, c, k))
    bias = rng.standard_normal(co)
    ref = torch.nn.functional.conv1d(torch.from_numpy(x), torch.from_numpy(w), torch.from_numpy(bias),
                                     stride=stride, padding=pad, dilation=dil).numpy()
    got = O.conv1d_ref(x, w.reshape(co, c * k), bias, k, stride, pad, dil)
    assert got.shape == ref.shape
    np.testing.assert_allclose(got, ref, rtol=1e-12, atol=1e-12)
    assert O.conv1d_out_len(length, k, stride, pad, dil) == ref.shape[2]


def test_conv1d_taps_column_order():
    x = np.arange(2 * 3 * 5, dtype=np.float64).reshape(2, 3, 5)
    taps = O.conv1d_taps(x, kernel=2, stride=1, padding=1, dilation=2)
    # row (b=1, t=2), column c * K + k = x[1, c, 2 + 2k - 1]: c=2, k=0 -> x[1, 2, 1]; k=1 -> x[1, 2, 3]
    lo = O.conv1d_out_len(5, 2, 1, 1, 2)
    assert taps[1 * lo + 2, 2 * 2 + 0] == x[1, 2, 1] and taps[1 * lo + 2, 2 * 2 + 1] == x[1, 2, 3]
    assert taps[0, 0] == 0.0  # t=0, k=0 reads position -1: zero padding


def test_snake_fixed_points_and_period():
    alpha = np.array([0.5, 1.0, 3.0])
    n = np.arange(-3, 4)[:, None]
    x = n * np.pi / alpha[None, :]                      # sin(alpha x) = 0
    np.testing.assert_allclose(O.snake_ref(x, alpha, channel_axis=1), x, atol=1e-12)
    rng = np.random.default_rng(0)
    x = rng.standard_normal((10, 3)) * 4
    y0 = O.snake_ref(x, alpha, channel_axis=1) - x
    y1 = O.snake_ref(x + np.pi / alpha, alpha, channel_axis=1) - (x + np.pi / alpha)
    np.testing.assert_allclose(y0, y1, atol=1e-9)
    assert (y0 >= 0).all() and (y0 <= 1.0 / alpha + 1e-12).all()
    # x = pi / (2 alpha): the added term is its maximum 1 / (alpha + eps)
    np.testing.assert_allclose(O.snake_ref(np.pi / (2 * alpha[None, :]), alpha, eps=0.0, channel_axis=1)
                               - np.pi / (2 * alpha), 1.0 / alpha[None, :], rtol=1e-12)


@pytest.mark.parametrize("k,stride,pad,opad", [(16, 8, 4, 0), (10, 5, 3, 0), (10, 5, 3, 1), (4, 2, 1, 0), (8, 4, 2, 0),
                                              (3, 1, 0, 0), (6, 3, 0, 0), (6, 3, 2, 1), (6, 3, 2, 2)])
def test_conv_transpose1d_ref_matches_torch(k, stride, pad, opad):
    rng = np.random.default_rng(k * 10 + stride + opad)
    b, ci, co, length = 2, 5, 4, 9
    x = rng.standard_normal((b, ci, length))
    w = rng.standard_normal((ci, co, k))
    bias = rng.standard_normal(co)
    ref = torch.nn.functional.conv_transpose1d(torch.from_numpy(x), torch.from_numpy(w), torch.from_numpy(bias),
                                               stride=stride, padding=pad, output_padding=opad).numpy()
    got = O.conv_transpose1d_ref(x, w.reshape(ci, co * k), bias, k, stride, pad, opad)
    assert got.shape == ref.shape
    np.testing.assert_allclose(got, ref, rtol=1e-12, atol=1e-12)


def test_decoder_block_lengths_match_the_reference_tensors():
    """Each upsampling block (kernel 2s, padding ceil(s/2), output padding s % 2) writes s outputs per input, so
    the strides 8, 5, 4, 2, 3 give the reference's target_len * 8, * 40, * 160, * 320, * 960 samples
    (src/models/quantized_omnivoice/tensors/audio_decode.py)."""
    import math

    from torch2vk_amd.omnivoice.decoder import AudioDecoderConfig, out_len

    expect = {8: 8, 5: 40, 4: 160, 2: 320, 3: 960}
    strides = (8, 5, 4, 2, 3)
    for t in (1, 2, 7, 75, 1000):
        length = t
        for s in strides:
            length = (length - 1) * s - 2 * math.ceil(s / 2) + 2 * s + s % 2
            assert length == t * expect[s]
        cfg = AudioDecoderConfig(codebooks=1, vocab=4, codebook_dim=8, latent=8, hidden=8, channels=64,
                                 strides=strides)
        assert out_len(cfg, t) == 960 * t


def test_cfg_score_ref_closed_forms():
    rng = np.random.default_rng(7)
    c_books, t_len, vocab, s_len = 2, 3, 11, 5
    logits = rng.standard_normal((2, s_len, c_books * vocab))
    mask_id = 4
    tokens = np.full(c_books * t_len, mask_id, np.int64)
    tokens[1] = 2                                            # an already decided position
    ct, cs = O.cfg_score_ref(logits, tokens, c_books, t_len, vocab, 0.0, 0.25, 0.0, 0, 0, mask_id)
    for c in range(c_books):
        for t in range(t_len):
            flat = c * t_len + t
            row = logits[0, s_len - t_len + t, c * vocab:(c + 1) * vocab]
            lp = row - np.log(np.exp(row).sum())              # guidance 0: the conditional log-probability
            lp_no_mask = lp.copy()
            lp_no_mask[mask_id] = -np.inf
            assert ct[flat] == int(np.argmax(lp_no_mask))
            want = lp_no_mask.max() - 0.25 * c
            assert (cs[flat] == -O.FLT_MAX) if flat == 1 else np.isclose(cs[flat], want, atol=1e-12)
    # guidance g: guided = (1 + g) c - g u, renormalised
    g = 1.5
    undecided = np.full(c_books * t_len, -1, np.int64)       # mask id -1: no token excluded, every position open
    ct, cs = O.cfg_score_ref(logits, undecided, c_books, t_len, vocab, g, 0.0, 0.0, 0, 0, -1)
    c_lp = logits[0, s_len - t_len][:vocab] - np.log(np.exp(logits[0, s_len - t_len][:vocab]).sum())
    u_lp = logits[1, 0][:vocab] - np.log(np.exp(logits[1, 0][:vocab]).sum())
    guided = (1 + g) * c_lp - g * u_lp
    assert ct[0] == int(np.argmax(guided))
    assert np.isclose(cs[0], guided.max() - np.log(np.exp(guided).sum()), atol=1e-12)


def _lowbias32_inverse(x: int) -> int:
    """The inverse of the lowbias32 integer hash (x ^= x >> 16; x *= 0x7feb352d; x ^= x >> 15;
    x *= 0x846ca68b; x ^= x >> 16), derived step by step: an odd multiplier is undone by its inverse mod 2^32,
    and x ^= x >> k by folding the shifted copies back in until they vanish."""
    def unxorshift(v: int, k: int) -> int:
        out, shifted = v, v >> k
        while shifted:
            out ^= shifted
            shifted >>= k
        return out & 0xFFFFFFFF
    x = unxorshift(x & 0xFFFFFFFF, 16)
    x = (x * pow(0x846CA68B, -1, 1 << 32)) & 0xFFFFFFFF
    x = unxorshift(x, 15)
    x = (x * pow(0x7FEB352D, -1, 1 << 32)) & 0xFFFFFFFF
    return unxorshift(x, 16)


def test_gumbel_hash_is_lowbias32():
    """The noise hash is the published lowbias32 mixer: composing it with the mixer's inverse is the identity,
    which a changed multiplier or shift in the oracle breaks; the inverse multipliers are the published ones."""
    assert pow(0x7FEB352D, -1, 1 << 32) == 0x1D69E2A5 and pow(0x846CA68B, -1, 1 << 32) == 0x43021123
    rng = np.random.default_rng(0)
    xs = list(range(4096)) + [int(v) for v in rng.integers(0, 1 << 32, 20000, dtype=np.uint64)] + [0xFFFFFFFF]
    for x in xs:
        assert _lowbias32_inverse(O.ov_hash(x)) == x, hex(x)
    # a planted mistake (one multiplier bit, one shift) is caught by the same composition
    def wrong(x: int, mult: int, shift: int) -> int:
        x ^= x >> 16
        x = (x * mult) & 0xFFFFFFFF
        x ^= x >> shift
        x = (x * 0x846CA68B) & 0xFFFFFFFF
        return x ^ (x >> 16)
    assert any(_lowbias32_inverse(wrong(x, 0x7FEB352F, 15)) != x for x in range(64))
    assert any(_lowbias32_inverse(wrong(x, 0x7FEB352D, 14)) != x for x in range(64))


def test_gumbel_noise_statistics():
    draws = np.array([O.ov_gumbel(1234, 7, i) for i in range(20000)])
    assert abs(draws.mean() - 0.5772156649) < 0.03          # the Gumbel mean is Euler's constant
    assert abs(draws.var() - np.pi ** 2 / 6) < 0.1
    assert O.ov_hash(0) == 0 and len({O.ov_hash(i) for i in range(5000)}) == 5000


def test_token_update_topk_ref_matches_sorting():
    rng = np.random.default_rng(3)
    c_books, t_len, s_len = 3, 4, 9
    scores = rng.standard_normal(c_books * t_len)
    scores[5] = scores[2]                                    # a tie: the lower index ranks first
    cand = rng.integers(0, 50, c_books * t_len)
    tokens = np.full(c_books * t_len, 99, np.int64)
    ids = np.full((2, c_books, s_len), -1, np.int64)
    new_tokens, new_ids = O.token_update_topk_ref(cand, scores, tokens, ids, 5)
    chosen = sorted(range(scores.size), key=lambda i: (-scores[i], i))[:5]
    assert set(np.nonzero(new_tokens != 99)[0]) == set(chosen)
    for i in chosen:
        c, t = divmod(i, t_len)
        assert new_ids[0, c, s_len - t_len + t] == cand[i] and new_ids[1, c, t] == cand[i]
    assert (new_ids != -1).sum() == 10


def test_unmask_schedule():
    from torch2vk_amd.omnivoice.generate import time_steps, unmask_schedule

    t = time_steps(0.0, 1.0, 8, 0.1)
    assert t[0] == 0.0 and abs(float(t[-1]) - 1.0) < 1e-7 and np.all(np.diff(t) > 0)
    assert abs(float(time_steps(0.0, 1.0, 2, 0.1)[1]) - 0.05 / 0.55) < 1e-7   # s t / (1 + (s - 1) t) at t = 1/2
    for total, steps in ((12, 4), (4000, 32), (7, 10)):
        sched = unmask_schedule(total, steps)
        assert len(sched) == steps and sum(sched) == total and min(sched) >= 0
    assert unmask_schedule(100, 4, t_shift=1.0) == [25, 25, 25, 25]           # no shift: an even split
    # float32 products (the reference's promotion): these totals round differently in float64
    # (..., 41, 125] and a 129 / 3894 pair)
    assert unmask_schedule(221, 8) == [4, 5, 6, 8, 12, 20, 40, 126]
    assert unmask_schedule(9752, 16)[5] == 128 and unmask_schedule(9752, 16)[-1] == 3895
    # fewer positions than steps: the remainder runs out and later steps unmask nothing
    sched = unmask_schedule(7, 10)
    assert sum(sched) == 7 and sched[-1] == 0 and all(k >= 0 for k in sched)
    assert unmask_schedule(100, 4)[0] < unmask_schedule(100, 4)[-1]           # shift 0.1: few early, many late
