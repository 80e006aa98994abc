"""GPU parity of the Qwen3-ASR audio tower: every new kernel against the CPU oracle or a library routine,
the whole tower against the oracle tower, and the audio-injected decode against the oracle decoder."""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle
from oracle import asr as oasr
from oracle import reference as R
from tests.conftest import assert_close

pytestmark = pytest.mark.gpu


def _bf16(a: np.ndarray) -> np.ndarray:
    return R.bf16_round(np.asarray(a, np.float32))


def _gelu64(x: np.ndarray) -> np.ndarray:
    return F.gelu(torch.from_numpy(np.asarray(x, np.float64))).numpy()


# (m, x columns, weight columns, n, bias, act, out): attention/MLP projections (both tile heights), the conv
# front-end shapes (K padded past the weight rows: 9 -> 32 of 64 and 4320 of 4352), a few rows
LINEAR_CASES = [
    (300, 896, 896, 896, True, None, "bf16"),
    (4100, 1024, 1024, 4096, True, "gelu", "bf16"),
    (3200, 64, 32, 480, True, "gelu", "bf16"),
    (517, 4352, 4320, 480, True, "gelu", "f32"),
    (40, 896, 896, 1024, True, None, "f32"),
    (130, 7680, 7680, 896, False, None, "f32"),
]


@pytest.mark.parametrize("splits", [1, None], ids=["one_pass", "auto_split"])
@pytest.mark.parametrize("m,kx,kw,n,bias,act,out", LINEAR_CASES)
def test_q8_0_linear_matches_oracle(device, m, kx, kw, n, bias, act, out, splits):
    """splits 1: the one-pass kernel; None: the wrapper's choice (small grids split K, the bias, GELU and
    residual then applied in the reduction)."""
    from torch2vk_amd import kernels

    print(f"q8_0_linear M={m} Kx={kx} Kw={kw} N={n} bias={bias} act={act} out={out} "
          f"splits={kernels.gemm_splits(m, n, kx) if splits is None else 1}", flush=True)
    rng = np.random.default_rng(m + kx + n)
    w = (rng.standard_normal((n, kw)) * 0.03).astype(np.float32)
    packed = oracle.quantize_q8_0(w)
    wd = oracle.dequant_q8_0(packed, kw)
    x = _bf16(rng.standard_normal((m, kx)))  # columns past kw are arbitrary finite values: they meet zeros
    b = (rng.standard_normal(n) * 0.5).astype(np.float32) if bias else None
    ref = x[:, :kw].astype(np.float64) @ _bf16(wd).astype(np.float64).T
    if b is not None:
        ref = ref + b
    if act == "gelu":
        ref = _gelu64(ref)
    xt = torch.from_numpy(x).to(device).to(torch.bfloat16)
    wt = torch.from_numpy(packed).to(device)
    bt = torch.from_numpy(b).to(device) if b is not None else None
    dt = torch.bfloat16 if out == "bf16" else torch.float32
    got = kernels.q8_0_linear(xt, wt, bias=bt, act=act, out_dtype=dt, splits=splits).float().cpu().numpy()
    scale = np.abs(ref).max()
    tol = 8e-3 * scale if out == "bf16" else 1e-5 * scale + 1e-5
    assert_close(got, ref, max_abs=tol, min_cos=0.99999, what="q8_0_linear")
    if out == "f32" and act is None:
        res = rng.standard_normal((m, n)).astype(np.float32)
        rt = torch.from_numpy(res).to(device)
        kernels.q8_0_linear(xt, wt, bias=bt, out=rt, residual=rt, splits=splits)
        assert_close(rt.cpu().numpy(), ref + res, max_abs=1e-5 * scale + 1e-5, min_cos=0.99999, what="residual")


def test_q8_0_linear_rejects_bad_shapes(device):
    from torch2vk_amd import kernels

    x = torch.zeros(4, 96, dtype=torch.bfloat16, device=device)
    w = torch.zeros(8, 34 * 3, dtype=torch.uint8, device=device)
    with pytest.raises(ValueError):
        kernels.q8_0_linear(x, w)  # K % 64
    x = torch.zeros(4, 64, dtype=torch.bfloat16, device=device)
    with pytest.raises(ValueError):
        kernels.q8_0_linear(x, w)  # weight rows longer than x's
    with pytest.raises(ValueError):
        kernels.q8_0_linear(x, w[:, :68], act="relu")


def test_im2col_matches_unfold(device):
    from torch2vk_amd import kernels

    g = torch.Generator().manual_seed(0)
    # fp32 mel chunks, NCHW
    x = torch.randn(3, 1, 128, 100, generator=g)
    got = kernels.im2col(x.to(device), (3, 3), (2, 2), (1, 1)).cpu()
    ref = F.unfold(x, 3, padding=1, stride=2).transpose(1, 2).reshape(-1, 9).to(torch.bfloat16)
    assert got.shape == (3 * 64 * 50, 64)
    assert torch.equal(got[:, :9], ref)
    assert not got[:, 9:].any()
    # bf16 channels-last activations
    y = torch.randn(2, 64, 50, 40, generator=g).to(torch.bfloat16)  # [B, H, W, C]
    got = kernels.im2col(y.to(device).permute(0, 3, 1, 2), (3, 3), (2, 2), (1, 1)).cpu()
    ref = F.unfold(y.permute(0, 3, 1, 2).float(), 3, padding=1, stride=2).transpose(1, 2).reshape(-1, 360)
    assert got.shape == (2 * 32 * 25, 384)
    assert torch.equal(got[:, :360].float(), ref)
    assert not got[:, 360:].any()
    # the (B, C*F, T) flatten + transpose before conv_out, as an (F x 1) patch
    z = torch.randn(2, 16, 13, 48, generator=g).to(torch.bfloat16)  # [B, F, T, C]
    got = kernels.im2col(z.to(device).permute(0, 3, 1, 2), (16, 1)).cpu()
    nchw = z.permute(0, 3, 1, 2)  # [B, C, F, T]
    ref = nchw.reshape(2, 48 * 16, 13).transpose(1, 2).reshape(-1, 768)
    assert torch.equal(got, ref)


@pytest.mark.parametrize("in_dtype,out_dtype", [(torch.float32, torch.bfloat16), (torch.float32, torch.float32),
                                                (torch.bfloat16, torch.bfloat16)])
def test_layer_norm_matches_closed_form(device, in_dtype, out_dtype):
    from torch2vk_amd import kernels

    g = torch.Generator().manual_seed(1)
    x = (torch.randn(301, 896, generator=g) * 4 + 2).to(in_dtype)
    w = torch.randn(896, generator=g) * 0.2 + 1
    b = torch.randn(896, generator=g) * 0.1
    got = kernels.layer_norm(x.to(device), w.to(device), b.to(device), out_dtype=out_dtype).float().cpu()
    ref = F.layer_norm(x.double(), (896,), w.double(), b.double(), eps=1e-5)
    tol = 2e-2 if out_dtype == torch.bfloat16 else 2e-5
    assert_close(got.numpy(), ref.numpy(), max_abs=tol, min_cos=0.99999, what="layer_norm")


def test_gelu_matches_closed_form(device):
    from torch2vk_amd import kernels

    x = torch.linspace(-8, 8, 4096)
    got = kernels.gelu(x.to(device)).cpu()
    assert_close(got.numpy(), _gelu64(x.numpy()), max_abs=2e-6, min_cos=0.999999, what="gelu fp32")
    got16 = kernels.gelu(x.to(torch.bfloat16).to(device)).float().cpu()
    ref16 = _gelu64(x.to(torch.bfloat16).float().numpy())
    assert_close(got16.numpy(), ref16, max_abs=4e-2, min_cos=0.9999, what="gelu bf16")


def test_row_gather_and_scatter(device):
    from torch2vk_amd import kernels

    g = torch.Generator().manual_seed(2)
    src = torch.randn(40, 96, generator=g)
    idx = torch.tensor([3, 0, 39, 3, 40, -1, 17])
    got = kernels.index_select_rows(src.to(device), idx.to(device)).cpu()
    assert torch.equal(got[[0, 1, 2, 3, 6]], src[idx[[0, 1, 2, 3, 6]]])
    assert not got[4].any() and not got[5].any()  # out of range -> zero rows
    dst = torch.randn(30, 96, generator=g)
    rows = torch.randn(4, 96, generator=g)
    pos = torch.tensor([29, 2, 30, 5])
    d = dst.to(device)
    kernels.index_copy_rows(d, pos.to(device), rows.to(device))
    ref = dst.clone()
    ref[[29, 2, 5]] = rows[[0, 1, 3]]  # index 30 is skipped
    assert torch.equal(d.cpu(), ref)


def test_embedding_q8_0_is_exact(device):
    from torch2vk_amd import kernels

    rng = np.random.default_rng(3)
    table = (rng.standard_normal((500, 256)) * 0.05).astype(np.float32)
    packed = oracle.quantize_q8_0(table)
    deq = oracle.dequant_q8_0(packed, 256)
    ids = torch.tensor([0, 499, 17, 17, 500, -3])
    got = kernels.embedding_q8_0(torch.from_numpy(packed).to(device), ids.to(device), 256).cpu().numpy()
    np.testing.assert_array_equal(got[:4], deq[ids[:4].numpy()])
    assert not got[4:].any()


def _segments_ref(q, k, v, cu, scale):
    """fp32 CPU attention window by window over [B, T, H, D] bf16-exact inputs (GQA by repetition)."""
    b, t, nh, d = q.shape
    nk = k.shape[2]
    kk = k.repeat_interleave(nh // nk, dim=2)
    vv = v.repeat_interleave(nh // nk, dim=2)
    out = torch.zeros(b, t, nh, d)
    for i in range(b):
        o = oasr.windowed_attention(q[i].float().transpose(0, 1), kk[i].float().transpose(0, 1),
                                    vv[i].float().transpose(0, 1), cu, scale)
        out[i] = o.transpose(0, 1)
    return out


SEG_CASES = [
    (1, 250, 14, 14, 64, [0, 104, 208, 250]),
    (2, 1500, 16, 16, 64, [0, 1500]),
    (1, 300, 4, 4, 128, [0, 1, 2, 3, 50, 51, 177, 300]),
    (1, 129, 2, 2, 64, [0, 129]),
    (1, 200, 8, 2, 64, [0, 64, 128, 192, 200]),
    # segments that start off the 64-key and 128-query grid, several tiles each (the C5 job's utterances)
    (1, 3000, 4, 4, 64, [0, 1500, 3000]),
    (1, 1000, 4, 2, 64, [0, 100, 700, 1000]),
    (1, 700, 2, 2, 128, [0, 300, 700]),
]


@pytest.mark.parametrize("b,t,nh,nk,d,cu", SEG_CASES)
def test_flash_attn_segments_matches_windowed_attention(device, b, t, nh, nk, d, cu):
    from torch2vk_amd import kernels

    print(f"flash_attn_segments b={b} t={t} nh={nh} nk={nk} d={d} segments={len(cu) - 1}", flush=True)
    g = torch.Generator().manual_seed(t + nh)
    q = torch.randn(b, t, nh, d, generator=g).to(torch.bfloat16)
    k = torch.randn(b, t, nk, d, generator=g).to(torch.bfloat16)
    v = torch.randn(b, t, nk, d, generator=g).to(torch.bfloat16)
    scale = d ** -0.5
    got = kernels.flash_attn_segments(q.to(device), k.to(device), v.to(device), cu).float().cpu()
    ref = _segments_ref(q, k, v, cu, scale)
    assert_close(got.numpy(), ref.numpy(), max_abs=2e-2, min_cos=0.9999, what="segments vs oracle")
    # the dense-mask kernel under the equivalent block-diagonal mask agrees with it
    from torch2vk_amd.qwen3_asr.preprocess import block_diagonal_mask

    mask = torch.from_numpy(block_diagonal_mask(np.array(cu))[0]).to(device)
    dense = kernels.flash_attn_prefill(q.to(device), k.to(device), v.to(device), causal=False, mask=mask)
    assert_close(got.numpy(), dense.float().cpu().numpy(), max_abs=2e-2, min_cos=0.9999, what="segments vs mask")


def test_flash_attn_segments_strided_qkv_and_uncovered_tokens(device):
    """q|k|v as column blocks of one [T, 3D] buffer (the encoder's fused projection); tokens outside the
    bounds get zeros."""
    from torch2vk_amd import kernels

    t, nh, d = 150, 4, 64
    g = torch.Generator().manual_seed(9)
    qkv = torch.randn(t, 3 * nh * d, generator=g).to(torch.bfloat16)
    dev = qkv.to(device)
    views = [dev[:, i * nh * d:(i + 1) * nh * d].view(1, t, nh, d) for i in range(3)]
    cu = torch.tensor([0, 60, 100], dtype=torch.int32, device=device)  # device table: taken as is
    got = kernels.flash_attn_segments(*views, cu).float().cpu()
    cpu = [qkv[:, i * nh * d:(i + 1) * nh * d].view(1, t, nh, d) for i in range(3)]
    ref = _segments_ref(cpu[0][:, :100], cpu[1][:, :100], cpu[2][:, :100], [0, 60, 100], d ** -0.5)
    assert_close(got[:, :100].numpy(), ref.numpy(), max_abs=2e-2, min_cos=0.9999, what="strided")
    assert not got[:, 100:].any()
    # tokens before the first bound see nothing either
    cu = torch.tensor([20, 60, 100], dtype=torch.int32, device=device)
    got = kernels.flash_attn_segments(*views, cu).float().cpu()
    ref = _segments_ref(cpu[0][:, 20:100], cpu[1][:, 20:100], cpu[2][:, 20:100], [0, 40, 80], d ** -0.5)
    assert_close(got[:, 20:100].numpy(), ref.numpy(), max_abs=2e-2, min_cos=0.9999, what="head gap")
    assert not got[:, :20].any() and not got[:, 100:].any()


def _tower(cfg, device, seed, frames, n_window_infer=None):
    from dataclasses import replace

    from torch2vk_amd.qwen3_asr import preprocess as pp
    from torch2vk_amd.qwen3_asr.encoder import (Qwen3AudioEncoder, audio_tensor_shapes, quantize_audio_weights,
                                                synthetic_audio_dense)

    if n_window_infer is not None:
        cfg = replace(cfg, n_window_infer=n_window_infer)
    dense = synthetic_audio_dense(cfg, seed=seed)
    weights = quantize_audio_weights(dense, cfg, device)
    rng = np.random.default_rng(seed)
    mel = rng.standard_normal((1, cfg.mel_bins, frames)).astype(np.float32)
    inp = pp.preprocess_audio_inputs(np.zeros(0), mel, np.ones(frames), cfg)
    enc = Qwen3AudioEncoder(weights)
    got = enc.run_audio_encoder(torch.from_numpy(inp["padded_feature"]).to(device),
                                torch.from_numpy(inp["position_embedding"]).to(device),
                                torch.from_numpy(inp["compact_index"]).to(device), inp["cu_seqlens"])
    oracle_w = oasr.dense_from_packed({k: v.cpu().numpy() for k, v in weights.packed.items()},
                                      {k: v.cpu().numpy() for k, v in weights.vectors.items()},
                                      audio_tensor_shapes(cfg))
    ref = oasr.audio_tower_cpu(oracle_w, cfg, inp["padded_feature"], inp["position_embedding"],
                               inp["compact_index"], cu_seqlens=inp["cu_seqlens"])
    return got.cpu(), ref, inp


def test_audio_tower_tiny_matches_oracle(device):
    from torch2vk_amd.qwen3_asr.config import AudioEncoderConfig

    cfg = AudioEncoderConfig(d_model=128, layers=2, heads=2, ffn=256, output_dim=128, conv_channels=32)
    got, ref, inp = _tower(cfg, device, seed=5, frames=260, n_window_infer=200)
    assert inp["cu_seqlens"].tolist() == [0, 26, 34]
    print(f"tiny tower: tokens {got.shape[0]}", flush=True)
    scale = float(ref.abs().max())
    assert_close(got.numpy(), ref.numpy(), max_abs=3e-2 * scale, min_cos=0.999, what="tiny tower")


def test_audio_tower_qwen3_asr_0_6b_shape(device):
    """The real tower shape (18 layers, 896 wide, 480-channel convs) on 10 s of frames: 130 tokens in windows
    of 104."""
    from torch2vk_amd.qwen3_asr.config import QWEN3_ASR_0_6B_AUDIO

    got, ref, inp = _tower(QWEN3_ASR_0_6B_AUDIO, device, seed=6, frames=1000)
    assert got.shape == (130, 1024) and inp["cu_seqlens"].tolist() == [0, 104, 130]
    scale = float(ref.abs().max())
    print(f"0.6B tower: max |ref| {scale:.3f}", flush=True)
    assert_close(got.numpy(), ref.numpy(), max_abs=5e-2 * scale, min_cos=0.999, what="0.6B tower")


def test_audio_injected_decode_matches_oracle(device):
    """Encoder features injected at the audio placeholder positions of the prompt embeddings, then greedy
    decode (Q8_0 token embedding as under the Qwen3-ASR policy): tokens equal the oracle decoder's given the
    same injected embeddings."""
    from oracle.qwen3_check import check_greedy_tokens, decoder_step_logits, dense_weights
    from oracle.reference import Qwen3Shape
    from torch2vk_amd.qwen3.config import Qwen3Config
    from torch2vk_amd.qwen3.model import Qwen3Decoder
    from torch2vk_amd.qwen3.weights import matrix_shapes, synthetic_weights
    from torch2vk_amd.qwen3_asr.config import AudioEncoderConfig
    from torch2vk_amd.qwen3_asr.encoder import run_audio_inject

    tcfg = Qwen3Config("tiny-asr", hidden=1024, layers=2, heads=8, kv_heads=2, head_dim=128, mlp=1024, vocab=1024,
                       eos_token_ids=(1023,))
    w = synthetic_weights(tcfg, device=device, seed=7, std=0.05, norm_std=0.1, policy="qwen3_asr")
    assert w.types["embed"] == "q8_0"
    acfg = AudioEncoderConfig(d_model=128, layers=1, heads=2, ffn=256, output_dim=1024, conv_channels=32)
    feats, _, _ = _tower(acfg, device, seed=8, frames=120)  # 16 audio tokens
    feats = feats.to(device)
    n_audio = feats.shape[0]
    prompt = [5, 6] + [900] * n_audio + [7, 8]  # placeholder id in-vocabulary for the tiny model
    positions = torch.arange(2, 2 + n_audio, device=device)
    dec = Qwen3Decoder(w, max_positions=64, max_new_tokens=16)
    dec.stop_on_eos = False
    embeds = dec.embed_tokens(torch.tensor(prompt, device=device))
    run_audio_inject(embeds, positions, feats)
    assert torch.equal(embeds[2:2 + n_audio], feats)
    toks = dec.generate_from_embeds(embeds, 10, steps_per_graph=4)
    print(f"asr decode: {toks}", flush=True)
    dense = dense_weights({k: v.cpu().numpy() for k, v in w.packed.items()}, w.types,
                          {k: v.cpu().numpy() for k, v in w.norms.items()}, matrix_shapes(tcfg))
    shape = Qwen3Shape(hidden=tcfg.hidden, layers=tcfg.layers, heads=tcfg.heads, kv_heads=tcfg.kv_heads,
                       head_dim=tcfg.head_dim, mlp=tcfg.mlp, vocab=tcfg.vocab, rope_theta=tcfg.rope_theta)
    print(check_greedy_tokens(shape, dense, prompt, toks, prompt_embeds=embeds.cpu(),
                              kv_history=(dec.k_cache, dec.v_cache), gpu_logits=decoder_step_logits(dec),
                              label="asr inject"))
