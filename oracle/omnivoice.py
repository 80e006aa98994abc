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
* cfg_score_ref, token_update_topk_ref and input_embed_ref follow OMNIVOICE_CFG_SCORE_F32,
  OMNIVOICE_TOKEN_UPDATE_TOPK_F32 and OMNIVOICE_INPUT_EMBED_Q8_0_F32 (src/models/quantized_omnivoice/shaders/
  omnivoice_*.py), the Gumbel hash bit for bit (lowbias32 constants).  Pinned in tests/test_omnivoice_host.py:
  the score against scipy-free log-softmax closed forms (guidance 0 = the conditional log-probability of the
  argmax), the noise by the Gumbel mean (Euler's constant), the ranking against a stable argsort.
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
                         padding: int = 0, output_padding: int = 0) -> np.ndarray:
    """x [B, Ci, L], w [Ci, Co * K] (row ci, element co * K + k) -> [B, Co, Lo] in float64, Lo = (L - 1) stride -
    2 padding + K + output_padding: every input i adds W[ci, co, k] x[b, ci, i] to output i * stride + k - padding;
    the output_padding positions at the end take whatever taps reach them (torch's conv_transpose1d)."""
    x = np.asarray(x, np.float64)
    b, ci, length = x.shape
    wk = np.asarray(w, np.float64).reshape(ci, -1, kernel)                 # [Ci, Co, K]
    co = wk.shape[1]
    full = np.zeros((b, co, (length - 1) * stride + kernel + output_padding))
    contrib = np.einsum("bci,cok->boik", x, wk)                             # [B, Co, L, K]
    for k in range(kernel):
        full[:, :, k:k + (length - 1) * stride + 1:stride] += contrib[:, :, :, k]
    lo = (length - 1) * stride - 2 * padding + kernel + output_padding
    y = full[:, :, padding:padding + lo]
    if bias is not None:
        y = y + np.asarray(bias, np.float64)[None, :, None]
    return y


FLT_MAX = float(np.finfo(np.float32).max)


def ov_hash(x: int) -> int:
    x &= 0xFFFFFFFF
    x ^= x >> 16
    x = (x * 0x7FEB352D) & 0xFFFFFFFF
    x ^= x >> 15
    x = (x * 0x846CA68B) & 0xFFFFFFFF
    x ^= x >> 16
    return x


def ov_gumbel(seed: int, step: int, flat: int) -> float:
    x = (seed ^ ((step * 0x9E3779B9) & 0xFFFFFFFF) ^ ((flat * 0x85EBCA6B) & 0xFFFFFFFF)) & 0xFFFFFFFF
    u = (float(ov_hash(x) & 0x00FFFFFF) + 0.5) * (1.0 / 16777216.0)
    u = min(max(u, 1.0e-7), 1.0 - 1.0e-7)
    return -np.log(-np.log(u))


def _log_softmax(v: np.ndarray) -> np.ndarray:
    m = v.max()
    return v - m - np.log(np.exp(v - m).sum())


def cfg_score_ref(logits: np.ndarray, tokens: np.ndarray, codebooks: int, targets: int, vocab: int, guidance: float,
                  layer_penalty: float, temperature: float, step: int, seed: int, mask_id: int):
    """logits [2, S, C * V] -> (candidate tokens [C * T], scores [C * T]) in float64."""
    lg = np.asarray(logits, np.float64)
    s_len = lg.shape[1]
    ct = np.zeros(codebooks * targets, np.int64)
    cs = np.zeros(codebooks * targets)
    for c in range(codebooks):
        for t in range(targets):
            flat = c * targets + t
            clp = _log_softmax(lg[0, s_len - targets + t, c * vocab:(c + 1) * vocab])
            ulp = _log_softmax(lg[1, t, c * vocab:(c + 1) * vocab])
            g = clp + guidance * (clp - ulp)
            cand = g.copy()
            if 0 <= mask_id < vocab:
                cand[mask_id] = -np.inf
            best = int(np.argmax(cand))              # first maximum: ties to the lowest id
            conf = g[best] - g.max() - np.log(np.exp(g - g.max()).sum()) - c * layer_penalty
            if temperature > 0:
                conf = conf / temperature + ov_gumbel(seed, step, flat)
            if tokens[flat] != mask_id:
                conf = -FLT_MAX
            ct[flat], cs[flat] = best, conf
    return ct, cs


def token_update_topk_ref(cand_tokens, cand_scores, tokens, batch_input_ids, unmask_count: int):
    """In place on copies: the min(unmask_count, C T) best (score desc, index asc) positions take their token."""
    tokens = np.array(tokens, copy=True)
    ids = np.array(batch_input_ids, copy=True)
    _, c_books, s_len = ids.shape
    n = tokens.size
    t_len = n // c_books
    order = np.argsort(-np.asarray(cand_scores, np.float64), kind="stable")
    for i in order[:min(unmask_count, n)]:
        c, t = divmod(int(i), t_len)
        tokens[i] = cand_tokens[i]
        ids[0, c, s_len - t_len + t] = cand_tokens[i]
        ids[1, c, t] = cand_tokens[i]
    return tokens, ids


def input_embed_ref(text_dense: np.ndarray, audio_dense: np.ndarray, ids: np.ndarray, audio_mask: np.ndarray,
                    vocab: int) -> np.ndarray:
    """text_dense [n_text, H], audio_dense [C * V, H] (dequantized rows) -> [B, S, H]."""
    b, c_books, s_len = ids.shape
    out = np.zeros((b, s_len, text_dense.shape[1]))
    for bi in range(b):
        for s in range(s_len):
            if audio_mask[bi, s]:
                for c in range(c_books):
                    tok = int(ids[bi, c, s])
                    if 0 <= tok < vocab:
                        out[bi, s] += audio_dense[c * vocab + tok]
            else:
                tok = int(ids[bi, 0, s])
                if 0 <= tok < text_dense.shape[0]:
                    out[bi, s] = text_dense[tok]
    return out


def audio_decode_ref(cfg, dense: dict, codes: np.ndarray, round_gemm_inputs=None) -> np.ndarray:
    """The acoustic decoder in float64 over dequantized weights (dense[name] as the GPU path uses them),
    following run_audio_decode (src/models/quantized_omnivoice/dispatch/audio_decode.py:60-760): codebook
    lookups and projections summed, fc2, conv1, per block snake -> conv_transpose1d -> residual units at
    dilations 1/3/9, snake -> conv2.  ``round_gemm_inputs`` (e.g. bf16 rounding) is applied where the GPU
    stages a GEMM's activations.  codes [C, T] -> waveform [T_out]."""
    x = audio_decode_front_ref(cfg, dense, codes, round_gemm_inputs)
    for i in range(len(cfg.strides)):
        x = audio_decode_block_ref(cfg, dense, x, i, round_gemm_inputs)
    return audio_decode_final_ref(dense, x, round_gemm_inputs)


def audio_decode_front_ref(cfg, dense: dict, codes: np.ndarray, round_gemm_inputs=None) -> np.ndarray:
    """Codebook lookups + projections summed, fc2, conv1 (audio_decode.py:66-149): [1, channels, T]."""
    rnd = round_gemm_inputs or (lambda a: a)
    t = codes.shape[1]
    acc = np.zeros((t, cfg.latent))
    for c in range(cfg.codebooks):
        e = dense[f"cb{c}"][codes[c]]
        acc = acc + rnd(e) @ dense[f"proj{c}.w"].T + dense[f"proj{c}.b"]
    h = rnd(acc) @ dense["fc2.w"].T + dense["fc2.b"]                     # [T, hidden]
    return conv1d_ref(rnd(h.T[None]), dense["conv1.w"], dense["conv1.b"], 7, 1, 3)   # [1, C, T]


def audio_decode_block_ref(cfg, dense: dict, x: np.ndarray, i: int, round_gemm_inputs=None) -> np.ndarray:
    """Upsampling block i (audio_decode.py:151-740): snake -> conv_transpose1d -> residual units at dilations
    1, 3, 9.  x [1, C, T] -> [1, C / 2, T']."""
    x = audio_decode_upsample_ref(cfg, dense, x, i)
    for j, d in enumerate((1, 3, 9)):
        x = audio_decode_unit_ref(dense, x, f"b{i}.r{j}.", d, round_gemm_inputs)
    return x


def audio_decode_upsample_ref(cfg, dense: dict, x: np.ndarray, i: int) -> np.ndarray:
    """snake -> conv_transpose1d of block i (kernel 2s, stride s, padding ceil(s/2), output padding s % 2)."""
    import math
    s = cfg.strides[i]
    x = snake_ref(np.asarray(x, np.float64), dense[f"b{i}.alpha"])
    return conv_transpose1d_ref(x, dense[f"b{i}.convt.w"], dense[f"b{i}.convt.b"], 2 * s, s, math.ceil(s / 2), s % 2)


def audio_decode_unit_ref(dense: dict, x: np.ndarray, p: str, d: int, round_gemm_inputs=None) -> np.ndarray:
    """One residual unit: x + conv_k1(snake(conv_k7,dilation d(snake(x))))."""
    rnd = round_gemm_inputs or (lambda a: a)
    x = np.asarray(x, np.float64)
    r = conv1d_ref(rnd(snake_ref(x, dense[p + "a1"])), dense[p + "c1.w"], dense[p + "c1.b"], 7, 1, 3 * d, d)
    return x + conv1d_ref(rnd(snake_ref(r, dense[p + "a2"])), dense[p + "c2.w"], dense[p + "c2.b"], 1)


def audio_decode_final_ref(dense: dict, x: np.ndarray, round_gemm_inputs=None) -> np.ndarray:
    """snake -> conv2 (audio_decode.py:741-755): the waveform [T_out]."""
    rnd = round_gemm_inputs or (lambda a: a)
    x = snake_ref(np.asarray(x, np.float64), dense["final.alpha"])
    return conv1d_ref(rnd(x), dense["conv2.w"], dense["conv2.b"], 7, 1, 3).reshape(-1)
