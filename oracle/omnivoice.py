"""CPU restatement of OmniVoice audio-decoder operators (test infrastructure only: the checker for the HIP
path, never called by it).

* conv1d_ref follows CONV1D_Q8_0W_F32B_F32 (src/models/quantized_omnivoice/shaders/conv1d_q8_0w_f32b_f32.py:
  conv_input_value -- input position t * stride + kh * dilation - padding, zero outside -- and the weight row
  of output channel co over the flattened (ic, kh) index k = ic * Kh + kh, plus the fp32 bias).  Pinned in
  tests/test_omnivoice_host.py against torch.nn.functional.conv1d.
* conv_transpose1d_ref follows CONV_TRANSPOSE1D_Q8_0W_F32B_F32 (src/models/quantized_omnivoice/shaders/
  conv_transpose1d_q8_0w_f32b_f32.py: deconv_input_value / deconv_weight_value -- output t takes input i
  through tap k when t + padding - k = i * stride; weight row ci, element co * Kh + k), as a scatter over the
  inputs.  Pinned against torch.nn.functional.conv_transpose1d.
* snake_ref follows the decoder's snake built from ADD_SCALAR (eps 1e-9), RECIPROCAL_F32, MUL_BROADCAST,
  SIN_F32, POW_SCALAR_F16 and ADD (src/models/quantized_omnivoice/dispatch/audio_decode.py:151-161), in
  float64 (the reference stores sin^2 in fp16; here it is kept exact).  Pinned by its fixed points
  (sin(alpha x) = 0 gives x) and its period pi / alpha in the added term.
"""

from __future__ import annotations

import numpy as np


def conv1d_out_len(length: int, kernel: int, stride: int = 1, padding: int = 0, dilation: int = 1) -> int:
    return (length + 2 * padding - dilation * (kernel - 1) - 1) // stride + 1


def conv1d_taps(x: np.ndarray, kernel: int, stride: int = 1, padding: int = 0, dilation: int = 1) -> np.ndarray:
    """x [B, C, L] -> [B * Lo, C * K] with column c * K + k = x[b, c, t * stride + k * dilation - padding]."""
    b, c, length = x.shape
    lo = conv1d_out_len(length, kernel, stride, padding, dilation)
    pos = np.arange(lo)[:, None] * stride + np.arange(kernel)[None, :] * dilation - padding      # [Lo, K]
    inside = (pos >= 0) & (pos < length)
    g = x[:, :, np.clip(pos, 0, length - 1)] * inside[None, None]                                  # [B, C, Lo, K]
    return g.transpose(0, 2, 1, 3).reshape(b * lo, c * kernel)


def conv1d_ref(x: np.ndarray, w: np.ndarray, bias: np.ndarray | None, kernel: int, stride: int = 1,
               padding: int = 0, dilation: int = 1) -> np.ndarray:
    """x [B, C, L], w [Co, C * K] (row co, column c * K + k) -> [B, Co, Lo] in float64."""
    b = x.shape[0]
    taps = conv1d_taps(np.asarray(x, np.float64), kernel, stride, padding, dilation)
    y = taps @ np.asarray(w, np.float64).T
    if bias is not None:
        y = y + np.asarray(bias, np.float64)[None, :]
    lo = taps.shape[0] // b
    return y.reshape(b, lo, -1).transpose(0, 2, 1)


def snake_ref(x: np.ndarray, alpha: np.ndarray, eps: float = 1e-9, channel_axis: int = 1) -> np.ndarray:
    """x + sin(alpha x)^2 / (alpha + eps), alpha per channel along ``channel_axis``."""
    x = np.asarray(x, np.float64)
    shape = [1] * x.ndim
    shape[channel_axis] = -1
    a = np.asarray(alpha, np.float64).reshape(shape)
    return x + np.sin(a * x) ** 2 / (a + eps)


def conv_transpose1d_ref(x: np.ndarray, w: np.ndarray, bias: np.ndarray | None, kernel: int, stride: int = 1,
                         padding: int = 0) -> np.ndarray:
    """x [B, Ci, L], w [Ci, Co * K] (row ci, element co * K + k) -> [B, Co, Lo] in float64, Lo = (L - 1) stride -
    2 padding + K: every input i adds W[ci, co, k] x[b, ci, i] to output i * stride + k - padding."""
    x = np.asarray(x, np.float64)
    b, ci, length = x.shape
    wk = np.asarray(w, np.float64).reshape(ci, -1, kernel)                 # [Ci, Co, K]
    co = wk.shape[1]
    full = np.zeros((b, co, (length - 1) * stride + kernel))
    contrib = np.einsum("bci,cok->boik", x, wk)                             # [B, Co, L, K]
    for k in range(kernel):
        full[:, :, k:k + (length - 1) * stride + 1:stride] += contrib[:, :, :, k]
    lo = (length - 1) * stride - 2 * padding + kernel
    y = full[:, :, padding:padding + lo]
    if bias is not None:
        y = y + np.asarray(bias, np.float64)[None, :, None]
    return y
