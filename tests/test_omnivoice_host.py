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


@pytest.mark.parametrize("k,stride,pad", [(16, 8, 4), (10, 5, 3), (4, 2, 1), (8, 4, 2), (3, 1, 0), (6, 3, 0)])
def test_conv_transpose1d_ref_matches_torch(k, stride, pad):
    rng = np.random.default_rng(k * 10 + stride)
    b, ci, co, length = 2, 5, 4, 9
    x = rng.standard_normal((b, ci, length))
    w = rng.standard_normal((ci, co, k))
    bias = rng.standard_normal(co)
    ref = torch.nn.functional.conv_transpose1d(torch.from_numpy(x), torch.from_numpy(w), torch.from_numpy(bias),
                                               stride=stride, padding=pad).numpy()
    got = O.conv_transpose1d_ref(x, w.reshape(ci, co * k), bias, k, stride, pad)
    assert got.shape == ref.shape
    np.testing.assert_allclose(got, ref, rtol=1e-12, atol=1e-12)
