"""GPU parity of the OmniVoice audio-decoder operators against oracle/omnivoice.py: the conv1d taps
(bit-exact), conv1d with Q8_0 weights at the decoder's kernel sizes and dilations, the snake activation, and
a whole residual unit (snake -> dilated conv k7 -> snake -> conv k1 -> + x)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from oracle import omnivoice as O
from oracle import reference as R
from tests.conftest import assert_close

pytestmark = pytest.mark.gpu


def _bf16(a: np.ndarray) -> np.ndarray:
    return R.bf16_round(np.asarray(a, np.float32)).astype(np.float64)


@pytest.mark.parametrize("k,stride,pad,dil", [(7, 1, 3, 1), (7, 1, 27, 9), (1, 1, 0, 1), (4, 3, 2, 2)])
def test_im2col_1d_bit_exact(device, k, stride, pad, dil):
    from torch2vk_amd import kernels

    rng = np.random.default_rng(k + 10 * dil)
    b, length, c = 2, 37, 24
    x = rng.standard_normal((b, length, c)).astype(np.float32)
    cols = kernels.im2col_1d(torch.from_numpy(x).to(device), k, stride=stride, padding=pad, dilation=dil)
    got = cols.float().cpu().numpy()
    ref = O.conv1d_taps(_bf16(x).transpose(0, 2, 1), k, stride, pad, dil)
    assert got.shape[0] == ref.shape[0] and got.shape[1] % 64 == 0
    assert np.array_equal(got[:, :c * k], ref)
    assert not got[:, c * k:].any()


@pytest.mark.parametrize("c,co,k,pad,dil", [(96, 64, 7, 3, 1), (64, 64, 7, 27, 9), (128, 96, 1, 0, 1)])
def test_conv1d_q8_0_matches_oracle(device, c, co, k, pad, dil):
    from torch2vk_amd import kernels

    rng = np.random.default_rng(c + co + dil)
    b, length = 2, 50
    x = rng.standard_normal((b, length, c)).astype(np.float32)
    w = (rng.standard_normal((co, c * k)) * 0.05).astype(np.float32)
    bias = rng.standard_normal(co).astype(np.float32)
    packed = kernels.quantize(torch.from_numpy(w).to(device), "q8_0")
    dense = oracle.dequant_q8_0(packed.cpu().numpy(), c * k)
    y = kernels.conv1d_q8_0(torch.from_numpy(x).to(device), packed, torch.from_numpy(bias).to(device), k,
                            padding=pad, dilation=dil)
    ref = O.conv1d_ref(_bf16(x).transpose(0, 2, 1), dense, bias, k, 1, pad, dil).transpose(0, 2, 1)
    got = y.cpu().numpy()
    print(f"conv1d c={c} co={co} k={k} dil={dil}: max-abs {np.abs(got - ref).max():.3e}", flush=True)
    # the GEMM stages dequantized weights as bf16: ~2^-9 relative per weight
    assert_close(got, ref, max_abs=1e-2 * float(np.abs(ref).max()), min_cos=0.9999, what="conv1d")


def test_snake_matches_oracle(device):
    from torch2vk_amd import kernels

    rng = np.random.default_rng(3)
    x = (rng.standard_normal((3, 41, 80)) * 3).astype(np.float32)
    alpha = np.abs(rng.standard_normal(80)).astype(np.float32) + 0.1
    y = kernels.snake(torch.from_numpy(x).to(device), torch.from_numpy(alpha).to(device)).cpu().numpy()
    ref = O.snake_ref(x, alpha, channel_axis=2)
    assert_close(y, ref, max_abs=2e-5 * float(np.abs(ref).max()), min_cos=0.9999999, what="snake")


@pytest.mark.parametrize("dil", [1, 3, 9])
def test_residual_unit_matches_oracle(device, dil):
    """The decoder's residual unit: y = x + conv_k1(snake2(conv_k7,dil(snake1(x)))), lengths preserved."""
    from torch2vk_amd import kernels

    rng = np.random.default_rng(20 + dil)
    b, length, c = 1, 64, 64
    x = rng.standard_normal((b, length, c)).astype(np.float32)
    a1, a2 = (np.abs(rng.standard_normal(c)).astype(np.float32) + 0.2 for _ in range(2))
    w1 = (rng.standard_normal((c, c * 7)) * 0.03).astype(np.float32)
    w2 = (rng.standard_normal((c, c)) * 0.1).astype(np.float32)
    b1, b2 = (rng.standard_normal(c).astype(np.float32) * 0.1 for _ in range(2))
    t = lambda a: torch.from_numpy(a).to(device)  # noqa: E731
    p1, p2 = kernels.quantize(t(w1), "q8_0"), kernels.quantize(t(w2), "q8_0")
    xd = t(x)
    s1 = kernels.snake(xd, t(a1))
    h1 = kernels.conv1d_q8_0(s1, p1, t(b1), 7, padding=3 * dil, dilation=dil)
    s2 = kernels.snake(h1, t(a2))
    y = kernels.conv1d_q8_0(s2, p2, t(b2), 1, residual=xd).cpu().numpy()
    d1, d2 = oracle.dequant_q8_0(p1.cpu().numpy(), c * 7), oracle.dequant_q8_0(p2.cpu().numpy(), c)
    xr = x.transpose(0, 2, 1).astype(np.float64)
    r1 = O.conv1d_ref(_bf16(O.snake_ref(xr, a1)), d1, b1, 7, 1, 3 * dil, dil)
    r2 = O.conv1d_ref(_bf16(O.snake_ref(r1, a2)), d2, b2, 1)
    ref = (xr + r2).transpose(0, 2, 1)
    assert y.shape == ref.shape
    print(f"residual unit dil={dil}: max-abs {np.abs(y - ref).max():.3e}", flush=True)
    assert_close(y, ref, max_abs=2e-2 * float(np.abs(ref).max()), min_cos=0.9999, what="residual unit")


@pytest.mark.parametrize("ci,co,k,stride,pad,opad", [(64, 32, 16, 8, 4, 0), (96, 48, 10, 5, 3, 0), (32, 32, 4, 2, 1, 0),
                                                     (48, 24, 3, 1, 0, 0), (96, 48, 10, 5, 3, 1), (64, 32, 6, 3, 2, 1)])
def test_conv_transpose1d_q8_0_matches_oracle(device, ci, co, k, stride, pad, opad):
    """The reference's Q8_0 rows [Ci, Co K] read as they are, fp32 arithmetic: agreement to fp32 rounding of
    the sums against the float64 oracle on the exactly dequantized weights."""
    from torch2vk_amd import kernels

    rng = np.random.default_rng(ci + k)
    b, length = 2, 21
    x = rng.standard_normal((b, length, ci)).astype(np.float32)
    # rows of Co K values in whole 32-value blocks (the last one zero-padded when Co K % 32 != 0)
    kk = co * k
    kpad = (kk + 31) // 32 * 32
    w = np.zeros((ci, kpad), np.float32)
    w[:, :kk] = rng.standard_normal((ci, kk)) * 0.05
    bias = rng.standard_normal(co).astype(np.float32)
    packed = kernels.quantize(torch.from_numpy(w).to(device), "q8_0")
    dense = oracle.dequant_q8_0(packed.cpu().numpy(), kpad)[:, :kk]
    y = kernels.conv_transpose1d_q8_0(torch.from_numpy(x).to(device), packed, torch.from_numpy(bias).to(device),
                                      co, k, stride=stride, padding=pad, output_padding=opad).cpu().numpy()
    ref = O.conv_transpose1d_ref(x.transpose(0, 2, 1), dense, bias, k, stride, pad, opad).transpose(0, 2, 1)
    assert y.shape[1] == (length - 1) * stride - 2 * pad + k + opad
    assert y.shape == ref.shape
    assert_close(y, ref, max_abs=1e-5 * float(np.abs(ref).max()), min_cos=0.9999999, what="conv_transpose1d")


def test_input_embed_matches_oracle(device):
    from torch2vk_amd import kernels

    rng = np.random.default_rng(9)
    b, c, s, h, vocab, n_text = 2, 3, 17, 64, 20, 50
    tw = (rng.standard_normal((n_text, h)) * 0.1).astype(np.float32)
    aw = (rng.standard_normal((c * vocab, h)) * 0.1).astype(np.float32)
    tp, ap = kernels.quantize(torch.from_numpy(tw).to(device), "q8_0"), kernels.quantize(torch.from_numpy(aw).to(device), "q8_0")
    ids = rng.integers(0, vocab, (b, c, s)).astype(np.int64)
    ids[0, 1, 3] = vocab + 5                     # outside the audio table: contributes 0
    mask = (rng.random((b, s)) < 0.6).astype(np.int32)
    got = kernels.omnivoice_input_embed_q8_0(tp, ap, torch.from_numpy(ids).to(device), torch.from_numpy(mask).to(device),
                                             vocab).cpu().numpy()
    ref = O.input_embed_ref(oracle.dequant_q8_0(tp.cpu().numpy(), h), oracle.dequant_q8_0(ap.cpu().numpy(), h), ids,
                            mask, vocab)
    assert_close(got, ref, max_abs=1e-6 * float(np.abs(ref).max()) + 1e-7, min_cos=0.9999999, what="input embed")


@pytest.mark.parametrize("temperature", [0.0, 5.0])
def test_cfg_score_matches_oracle(device, temperature):
    from torch2vk_amd import kernels

    rng = np.random.default_rng(11)
    c, t, s, vocab, mask_id = 8, 20, 30, 1025, 1024
    logits = (rng.standard_normal((2, s, c * vocab)) * 3).astype(np.float32)
    tokens = np.full(c * t, mask_id, np.int64)
    tokens[::7] = 3                              # decided positions score -FLT_MAX
    kw = dict(codebooks=c, targets=t, vocab=vocab, guidance=2.0, layer_penalty=0.1, temperature=temperature,
              step=3, seed=1234, mask_id=mask_id)
    ct, cs = kernels.omnivoice_cfg_score(torch.from_numpy(logits).to(device), torch.from_numpy(tokens).to(device), **kw)
    rt, rs = O.cfg_score_ref(logits, tokens, c, t, vocab, 2.0, 0.1, temperature, 3, 1234, mask_id)
    assert np.array_equal(ct.cpu().numpy(), rt)
    got = cs.cpu().numpy().astype(np.float64)
    open_ = tokens == mask_id
    assert np.all(got[~open_] == -O.FLT_MAX)
    assert np.abs(got[open_] - rs[open_]).max() <= 1e-3, np.abs(got[open_] - rs[open_]).max()


def test_token_update_topk_matches_oracle(device):
    from torch2vk_amd import kernels

    rng = np.random.default_rng(13)
    c, t, s = 8, 25, 40
    scores = rng.standard_normal(c * t).astype(np.float32)
    scores[[4, 9, 30]] = scores[17]              # ties go to the lower index
    scores[::11] = -O.FLT_MAX                    # decided positions never rank
    cand = rng.integers(0, 1024, c * t).astype(np.int64)
    tokens = np.full(c * t, 1024, np.int64)
    ids = rng.integers(0, 1024, (2, c, s)).astype(np.int64)
    td, idd = torch.from_numpy(tokens).to(device), torch.from_numpy(ids).to(device)
    kernels.omnivoice_token_update_topk(torch.from_numpy(cand).to(device), torch.from_numpy(scores).to(device), td, idd,
                                        unmask_count=37)
    rt, rids = O.token_update_topk_ref(cand, scores.astype(np.float64), tokens, ids, 37)
    assert np.array_equal(td.cpu().numpy(), rt)
    assert np.array_equal(idd.cpu().numpy(), rids)


@pytest.mark.parametrize("strides", [(2, 4), (8, 5, 4, 2, 3)])
def test_audio_decoder_matches_oracle(device, strides):
    """The whole acoustic decoder (2 codebooks, upsampling blocks of strides 2 and 4, and the reference's five
    blocks of strides 8, 5, 4, 2, 3 with 960 samples per frame) against the float64 oracle on the same
    dequantized weights, with GEMM activations and weights rounded to bf16 where the GPU stages them: stage by
    stage (conv1, each transposed conv, each residual unit, the output conv) over the GPU's own input to the
    stage, and end to end."""
    from torch2vk_amd.omnivoice.decoder import AudioDecoderConfig, OmniVoiceAudioDecoder, out_len, synthetic_dense

    cfg = AudioDecoderConfig(codebooks=2, vocab=16, codebook_dim=32, latent=64, hidden=64,
                             channels=128 if len(strides) == 2 else 512, strides=strides)
    dense = synthetic_dense(cfg, seed=5)
    dec = OmniVoiceAudioDecoder(cfg, dense, device)
    deq = {}
    for n, a in dense.items():
        if a.ndim == 2:
            kp = (a.shape[1] + 31) // 32 * 32
            deq[n] = oracle.dequant_q8_0(dec.w[n].cpu().numpy(), kp)[:, :a.shape[1]].astype(np.float64)
            # the GEMM-run ops (linears, conv1d) stage dequantized weights as bf16 (d q rounded to nearest
            # even); the embedding and conv_transpose1d read them in fp32
            if not (n.startswith("cb") or n.endswith("convt.w")):
                deq[n] = _bf16(deq[n])
        else:
            deq[n] = a.astype(np.float64)
    codes = np.random.default_rng(8).integers(0, cfg.vocab, (cfg.codebooks, 10)).astype(np.int64)
    stages = []
    y = dec.decode(torch.from_numpy(codes), stages=stages).cpu().numpy()
    ref = O.audio_decode_ref(cfg, deq, codes, round_gemm_inputs=_bf16)
    assert y.shape == (out_len(cfg, 10),) == ref.shape
    if strides == (8, 5, 4, 2, 3):
        assert y.shape == (960 * 10,)
    print(f"audio decoder: {y.shape[0]} samples, max-abs {np.abs(y - ref).max():.3e}, max |ref| {np.abs(ref).max():.3e}",
          flush=True)
    # every stage against the oracle run on the GPU's own input to that stage (its fp32 activations, staged to
    # bf16 by the oracle where the GPU's GEMMs stage them): each stage's error alone, with no amplification of
    # earlier roundings through later blocks
    to_ref = lambda a: a.cpu().numpy().astype(np.float64)[0].T[None]  # noqa: E731  channels-last -> [1, C, T]
    got_stage = [to_ref(a) for a in stages]
    checks = [("front", got_stage[0], O.audio_decode_front_ref(cfg, deq, codes, _bf16))]
    k = 1
    for i in range(len(strides)):
        checks.append((f"block {i} upsample", got_stage[k], O.audio_decode_upsample_ref(cfg, deq, got_stage[k - 1], i)))
        k += 1
        for j, d in enumerate((1, 3, 9)):
            want = O.audio_decode_unit_ref(deq, got_stage[k - 1], f"b{i}.r{j}.", d, _bf16)
            checks.append((f"block {i} unit {j}", got_stage[k], want))
            k += 1
    assert k == len(got_stage)
    checks.append(("final", y, O.audio_decode_final_ref(deq, got_stage[-1], _bf16)))
    rels = [float(np.abs(got - want).max()) / float(np.abs(want).max()) for _, got, want in checks]
    print("  stage max-abs / max: " + ", ".join(f"{w} {r:.1e}" for (w, _, _), r in zip(checks, rels)), flush=True)
    for what, got, want in checks:
        # one stage holds at most two GEMMs.  Stages where no staged bf16 rounding flips agree to ~1e-7 of their
        # maximum (fp32 summation order); a stage whose fp32 order flips the bf16 rounding of one snake output
        # (2^-8 of that value, through one conv's weights) measured up to 7e-4 of its maximum
        assert_close(got, want, max_abs=2e-3 * float(np.abs(want).max()), min_cos=0.99999, what=what)
    if len(strides) == 2:
        assert_close(y, ref, max_abs=1e-4 * float(np.abs(ref).max()), min_cos=0.9999999, what="waveform")
    else:
        # end to end, 5 blocks and 15 residual units amplify each stage's rounding (the float64 oracle itself
        # moves by 1.9 % of its maximum when its staged values are perturbed by 1e-7 relative): the waveform's
        # direction is held, the per-stage checks above hold its values
        assert_close(y, ref, max_abs=float("inf"), min_cos=0.999, what="waveform")


def test_generation_loop(device):
    """OmniVoice's loop on a 2-layer backbone: every step unmasks exactly the scheduled count, the two sequence
    copies carry the tokens, nothing stays masked; the first step's logits match the CPU oracle's masked
    Qwen3 pass and Q6_K head on the same embeddings."""
    from torch2vk_amd import kernels
    from torch2vk_amd.omnivoice.generate import OmniVoiceGenerator, unmask_schedule
    from torch2vk_amd.qwen3.config import Qwen3Config
    from torch2vk_amd.qwen3.model import Qwen3Decoder
    from torch2vk_amd.qwen3.weights import matrix_shapes, synthetic_weights
    from oracle.qwen3_check import dense_weights
    from oracle.reference import Qwen3Shape

    cfg = Qwen3Config("tiny-ov", hidden=1024, layers=2, heads=8, kv_heads=2, head_dim=128, mlp=1024, vocab=1024,
                      eos_token_ids=(1023,))
    w = synthetic_weights(cfg, device=device, seed=71, std=0.05, norm_std=0.1)
    llm = Qwen3Decoder(w, max_positions=32, max_new_tokens=4)
    c, v, mask_id, t_len, s_len = 2, 64, 63, 6, 16
    rng = np.random.default_rng(12)
    q = lambda a, wt: kernels.quantize(torch.from_numpy(a.astype(np.float32)).to(device), wt)  # noqa: E731
    text_w = q(rng.standard_normal((cfg.vocab, cfg.hidden)) * 0.05, "q8_0")
    audio_w = q(rng.standard_normal((c * v, cfg.hidden)) * 0.05, "q8_0")
    head_w = q(rng.standard_normal((c * v, cfg.hidden)) * 0.05, "q6_k")
    ids = np.zeros((2, c, s_len), np.int64)
    ids[0, :, :s_len - t_len] = rng.integers(0, cfg.vocab, s_len - t_len)
    ids[0, :, s_len - t_len:] = mask_id
    ids[1, :, :t_len] = mask_id
    amask = np.zeros((2, s_len), np.int32)
    amask[0, s_len - t_len:] = 1
    amask[1, :t_len] = 1
    attn = np.zeros((2, s_len, s_len), np.float32)
    attn[1, :t_len, t_len:] = -np.inf                # the unconditional targets see only themselves
    ids_d, amask_d, attn_d = (torch.from_numpy(a).to(device) for a in (ids, amask, attn))
    tokens = torch.full((c * t_len,), mask_id, dtype=torch.int64, device=device)
    gen = OmniVoiceGenerator(llm, text_w, audio_w, head_w, codebooks=c, vocab=v, mask_id=mask_id)
    # step-0 logits against the oracle on the same embeddings
    hidden = kernels.omnivoice_input_embed_q8_0(text_w, audio_w, ids_d, amask_d, v).cpu()
    lg0 = gen.logits(ids_d, amask_d, attn_d).cpu().numpy()
    dense = dense_weights({k: x.cpu().numpy() for k, x in w.packed.items()}, w.types,
                          {k: x.cpu().numpy() for k, x in w.norms.items()}, matrix_shapes(cfg))
    shape = Qwen3Shape(hidden=cfg.hidden, layers=cfg.layers, heads=cfg.heads, kv_heads=cfg.kv_heads,
                       head_dim=cfg.head_dim, mlp=cfg.mlp, vocab=cfg.vocab, rope_theta=cfg.rope_theta)
    head = oracle.dequant_q6_k(head_w.cpu().numpy(), cfg.hidden).astype(np.float64)
    for b in range(2):
        hb = R.Qwen3CpuModel(shape, dense, max_positions=32).forward(None, 0, embeds=hidden[b],
                                                                     mask=torch.from_numpy(attn[b]), all_positions=True)
        ref = hb.double().numpy() @ head.T
        assert_close(lg0[b], ref, max_abs=0.05 * float(np.abs(ref).max()), min_cos=0.999, what=f"logits row {b}")
    sched = unmask_schedule(c * t_len, 4)
    seen = []
    gen.generate(ids_d, amask_d, attn_d, tokens, num_steps=4, guidance=2.0, layer_penalty=0.1, temperature=0.0,
                 on_step=lambda step, k, lg: seen.append(int((tokens != mask_id).sum().item())))
    assert seen == list(np.cumsum(sched)), (seen, sched)
    tk = tokens.cpu().numpy()
    assert (tk != mask_id).all() and (tk >= 0).all() and (tk < v).all()
    out_ids = ids_d.cpu().numpy()
    for i in range(c * t_len):
        cb, t = divmod(i, t_len)
        assert out_ids[0, cb, s_len - t_len + t] == tk[i] == out_ids[1, cb, t]
