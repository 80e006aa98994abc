"""The persistent decode-layers kernel (t2h_qwen3_decode_layers) against the one-launch-per-op path
and the CPU oracle, at the Qwen3-8B layer shape (hidden 4096, MLP 12288, 32/8 heads), the Qwen3-0.6B
layer shape (hidden 1024, MLP 3072, 16/8 heads) and the Qwen3-1.7B layer shape (hidden 2048, MLP 6144,
16/8 heads), 2 layers each."""

from __future__ import annotations

from dataclasses import replace

import numpy as np
import pytest
import torch

from oracle.qwen3_check import check_greedy_tokens, decoder_step_logits, dense_weights
from oracle.reference import Qwen3Shape

pytestmark = pytest.mark.gpu


SHAPES = ["8b", "0.6b", "1.7b"]


def _base(name):
    from torch2vk_amd.qwen3.config import QWEN3_0_6B, QWEN3_1_7B, QWEN3_8B

    return {"8b": QWEN3_8B, "0.6b": QWEN3_0_6B, "1.7b": QWEN3_1_7B}[name]


@pytest.fixture(scope="module", params=SHAPES)
def setup_8b2(device, request):
    from torch2vk_amd.qwen3.weights import synthetic_weights

    base = _base(request.param)
    cfg = replace(base, layers=2, vocab=4096, eos_token_ids=(4095,))
    w = synthetic_weights(cfg, device=device, seed=7, std=0.02, norm_std=0.1)
    shape = Qwen3Shape(hidden=cfg.hidden, layers=cfg.layers, heads=cfg.heads, kv_heads=cfg.kv_heads,
                       head_dim=cfg.head_dim, mlp=cfg.mlp, vocab=cfg.vocab, rope_theta=cfg.rope_theta)
    return cfg, w, shape


# Workspace layout of decode_layers.hip: 256 B launch counter, then q|k|v as (fp32, u32 epoch) words,
# then the attention output as (bf16, u16 epoch) words.
WS_QKV = 256


def _ws_attn(cfg) -> int:
    return WS_QKV + (cfg.q_dim + 2 * cfg.kv_dim) * 8


def _ws_ll32(dec, offset, n):
    """fp32 values of n epoch-tagged (fp32, u32) words of the persistent kernel's workspace."""
    return dec.layers_ws[offset:offset + 8 * n].view(torch.int32).view(n, 2)[:, 0].contiguous().view(torch.float32)


def _ws_ll16(dec, offset, n):
    """bf16 values of n epoch-tagged (bf16, u16) words of the persistent kernel's workspace."""
    return dec.layers_ws[offset:offset + 4 * n].view(torch.int16).view(n, 2)[:, 0].contiguous().view(torch.bfloat16)


@pytest.mark.parametrize("pos", [0, 5, 255, 256, 300])
def test_persistent_layer_matches_per_op(device, setup_8b2, pos):
    """One layer at one position on random caches: the Q|K|V projections are bit-identical to the
    per-op GEMV (same lane mapping and reduction order); the attention output differs at most by
    bf16 rounding of a differently ordered fp32 sum; h by what that rounding does downstream.
    Positions 0, 5 and 255 (up to 256 keys) take the one-block-per-kv-head attention without a merge
    phase; 256 and 300 spread the keys over 32 blocks per kv head and merge."""
    from torch2vk_amd.qwen3.model import Qwen3Decoder

    cfg, w, _ = setup_8b2
    print(f"persistent vs per-op layer 0 at pos {pos}", flush=True)
    a = Qwen3Decoder(w, max_positions=512, max_new_tokens=4, persistent=True)
    b = Qwen3Decoder(w, max_positions=512, max_new_tokens=4, persistent=False)
    g = torch.Generator(device=device)
    g.manual_seed(3 + pos)
    kc = torch.randn(a.k_cache.shape, generator=g, device=device).to(torch.bfloat16)
    vc = torch.randn(a.v_cache.shape, generator=g, device=device).to(torch.bfloat16)
    h0 = torch.randn(cfg.hidden, generator=g, device=device)
    for d in (a, b):
        d.k_cache.copy_(kc)
        d.v_cache.copy_(vc)
        d.h.copy_(h0)
        d.position.fill_(pos)
    # run only layer 0 on both sides
    a.layer_table = a.layer_table[:1].contiguous()
    a.run_decode_layers()
    b.run_decode_layer(0)
    torch.cuda.synchronize()
    a.check_status()
    qkv = _ws_ll32(a, WS_QKV, cfg.q_dim + 2 * cfg.kv_dim)
    torch.testing.assert_close(qkv, torch.cat([b.q, b.k, b.v]), rtol=0, atol=0)
    attn = _ws_ll16(a, _ws_attn(cfg), cfg.q_dim).float()
    ref = b.attn.float()
    assert (attn - ref).abs().max().item() <= 2 ** -7 * ref.abs().max().item()
    torch.testing.assert_close(a.k_cache[0], b.k_cache[0], rtol=0, atol=0)
    torch.testing.assert_close(a.v_cache[0], b.v_cache[0], rtol=0, atol=0)
    # both attention outputs are within half a bf16 step of the fp64 value; where the two fp32 sums round
    # to neighbouring bf16 values, o_proj and the MLP carry that step into h
    herr = (a.h - b.h).abs().max().item()
    assert herr <= 3e-3 * b.h.abs().max().item(), herr


def test_persistent_prefill_close_to_per_op(device, setup_8b2):
    """Both layers over a 6-token prompt: the two paths differ only by rounding order."""
    from torch2vk_amd.qwen3.model import Qwen3Decoder

    cfg, w, _ = setup_8b2
    a = Qwen3Decoder(w, max_positions=128, max_new_tokens=16, persistent=True)
    b = Qwen3Decoder(w, max_positions=128, max_new_tokens=16, persistent=False)
    assert a.persistent and not b.persistent
    prompt = torch.tensor([17, 4000, 5, 999, 123, 64])
    for dec in (a, b):
        dec.stop_on_eos = False
        dec.prefill(prompt)
    torch.cuda.synchronize()
    a.check_status()
    ha, hb = a.h.double().cpu().numpy(), b.h.double().cpu().numpy()
    err = float(np.abs(ha - hb).max())
    cos = float(ha @ hb / np.linalg.norm(ha) / np.linalg.norm(hb))
    print(f"hidden after prefill: max-abs diff {err:.3e} (max |h| {np.abs(hb).max():.3e}), cos {cos:.8f}", flush=True)
    assert err <= 5e-3 * float(np.abs(hb).max()) and cos >= 0.99999


def test_persistent_decode_matches_oracle(device, setup_8b2):
    from torch2vk_amd.qwen3.model import Qwen3Decoder
    from torch2vk_amd.qwen3.weights import matrix_shapes

    cfg, w, shape = setup_8b2
    dense = dense_weights({k: v.cpu().numpy() for k, v in w.packed.items()}, w.types,
                          {k: v.cpu().numpy() for k, v in w.norms.items()}, matrix_shapes(cfg))
    prompt = np.random.default_rng(2).integers(0, cfg.vocab, 5).tolist()
    dec = Qwen3Decoder(w, max_positions=128, max_new_tokens=16, persistent=True)
    dec.stop_on_eos = False
    toks = dec.generate(torch.tensor(prompt), 10, steps_per_graph=4, use_graph=True)
    print(f"persistent {cfg.name}-shape decode: {toks}", flush=True)
    print(check_greedy_tokens(shape, dense, prompt, toks, kv_history=(dec.k_cache, dec.v_cache),
                              gpu_logits=decoder_step_logits(dec), label=f"persistent {cfg.name}"))


def test_persistent_graph_replay_equals_eager(device, setup_8b2):
    from torch2vk_amd.qwen3.model import Qwen3Decoder

    cfg, w, _ = setup_8b2
    prompt = torch.tensor([5, 9, 100, 7])
    a = Qwen3Decoder(w, max_positions=128, max_new_tokens=24, persistent=True)
    b = Qwen3Decoder(w, max_positions=128, max_new_tokens=24, persistent=True)
    a.stop_on_eos = b.stop_on_eos = False
    ta = a.generate(prompt, 17, use_graph=False)
    tb = b.generate(prompt, 17, steps_per_graph=4, use_graph=True)
    print(f"eager {ta}\ngraph {tb}", flush=True)
    assert ta == tb
    n = prompt.numel() + 17
    torch.testing.assert_close(a.k_cache[:, :n], b.k_cache[:, :n], rtol=0, atol=0)
    torch.testing.assert_close(a.v_cache[:, :n], b.v_cache[:, :n], rtol=0, atol=0)


# ------------------------------------------------------------------------------------------------------
# The benchmarked configurations: the 8B shape at a KV cache of 4096 positions and near the 8192 capacity
# (17 and 32 attention rows per wave), and the full 28-layer 0.6B decoder.


@pytest.fixture(scope="module")
def setup_8b_long(device):
    from torch2vk_amd.qwen3.config import QWEN3_8B
    from torch2vk_amd.qwen3.weights import matrix_shapes, synthetic_weights

    cfg = replace(QWEN3_8B, layers=2, vocab=4096, eos_token_ids=(4095,))
    w = synthetic_weights(cfg, device=device, seed=8, std=0.02, norm_std=0.1)
    shape = Qwen3Shape(hidden=cfg.hidden, layers=cfg.layers, heads=cfg.heads, kv_heads=cfg.kv_heads,
                       head_dim=cfg.head_dim, mlp=cfg.mlp, vocab=cfg.vocab, rope_theta=cfg.rope_theta)
    dense = dense_weights({k: v.cpu().numpy() for k, v in w.packed.items()}, w.types,
                          {k: v.cpu().numpy() for k, v in w.norms.items()}, matrix_shapes(cfg))
    return cfg, w, shape, dense


@pytest.mark.parametrize("pos", [4096, 8100])
def test_persistent_long_kv_matches_per_op(device, setup_8b_long, pos):
    """Layer 0 of the 8B shape at cache position 4096 (the headline bench: 17 rows per attention wave) and 8100
    (32 rows per wave, the kernel's limit) on an N(0,1) cache: q|k|v and the new K/V rows are bit-identical to
    the per-op kernels'; the attention output differs by at most bf16 rounding of a differently ordered sum."""
    from torch2vk_amd.qwen3.model import Qwen3Decoder

    cfg, w, _, _ = setup_8b_long
    print(f"persistent vs per-op, 8B shape, layer 0 at pos {pos}", flush=True)
    a = Qwen3Decoder(w, max_positions=8192, max_new_tokens=4, persistent=True)
    b = Qwen3Decoder(w, max_positions=8192, max_new_tokens=4, persistent=False)
    g = torch.Generator(device=device)
    g.manual_seed(pos)
    kc = torch.randn(a.k_cache.shape, generator=g, device=device).to(torch.bfloat16)
    vc = torch.randn(a.v_cache.shape, generator=g, device=device).to(torch.bfloat16)
    h0 = torch.randn(cfg.hidden, generator=g, device=device)
    for d in (a, b):
        d.k_cache.copy_(kc)
        d.v_cache.copy_(vc)
        d.h.copy_(h0)
        d.position.fill_(pos)
    del kc, vc
    a.layer_table = a.layer_table[:1].contiguous()
    a.run_decode_layers()
    b.run_decode_layer(0)
    torch.cuda.synchronize()
    a.check_status()
    assert int(a.status.item()) == 0
    qkv = _ws_ll32(a, WS_QKV, cfg.q_dim + 2 * cfg.kv_dim)
    torch.testing.assert_close(qkv, torch.cat([b.q, b.k, b.v]), rtol=0, atol=0)
    torch.testing.assert_close(a.k_cache[0], b.k_cache[0], rtol=0, atol=0)
    torch.testing.assert_close(a.v_cache[0], b.v_cache[0], rtol=0, atol=0)
    attn = _ws_ll16(a, _ws_attn(cfg), cfg.q_dim).float()
    ref = b.attn.float()
    err = (attn - ref).abs().max().item()
    print(f"attention max-abs diff {err:.3e} (max {ref.abs().max().item():.3e})", flush=True)
    assert err <= 2 ** -7 * ref.abs().max().item()
    # as in test_persistent_layer_matches_per_op: neighbouring bf16 roundings of the attention output carried
    # through o_proj and the MLP
    herr = (a.h - b.h).abs().max().item()
    assert herr <= 3e-3 * b.h.abs().max().item(), herr


def test_persistent_long_kv_decode_matches_oracle(device, setup_8b_long):
    """Greedy decode with the persistent kernel from an N(0,1) KV cache of 4096 positions (the headline bench's
    state): a 2-token prompt at positions 4096-4097, then 8 tokens through graph replay; every token against the
    CPU oracle started from the same cache, and the kernel's status word stays clear."""
    from torch2vk_amd.qwen3.model import Qwen3Decoder

    cfg, w, shape, dense = setup_8b_long
    start = 4096
    dec = Qwen3Decoder(w, max_positions=start + 64, max_new_tokens=16, persistent=True)
    dec.stop_on_eos = False
    g = torch.Generator(device=device)
    g.manual_seed(41)
    dec.k_cache[:, :start].normal_(generator=g)
    dec.v_cache[:, :start].normal_(generator=g)
    prompt = [77, 3001]
    print(f"persistent 8B-shape decode from KV {start}", flush=True)
    dec.prefill(torch.tensor(prompt), start=start)
    dec.run_steps(7, steps_per_graph=4, use_graph=True)
    toks = dec.generated[:int(dec.length.item())].tolist()
    dec.check_status()
    assert int(dec.status.item()) == 0 and len(toks) == 8
    print(f"tokens {toks}", flush=True)
    kv = (dec.k_cache[:, :start].cpu(), dec.v_cache[:, :start].cpu())
    stats = check_greedy_tokens(shape, dense, prompt, toks, start=start, kv_init=kv,
                                kv_history=(dec.k_cache, dec.v_cache), gpu_logits=decoder_step_logits(dec),
                                label="persistent 8B from KV 4096")
    print(stats, flush=True)


@pytest.mark.parametrize("policy", ["uniform", "q4_k_m"])
def test_persistent_0_6b_full_depth_matches_oracle(device, policy):
    """The whole 28-layer Qwen3-0.6B decoder (vocab 151936) in the persistent kernel: a 128-token random prompt
    fed one launch per position, then 32 greedy tokens in HIP graphs; status clear after all 160 launches and
    every token against the CPU oracle.  This depth is where residual hold threads once polled rows owned by
    another block and a bounded wait gave up.  Q4_K_M: 14 of the 28 layers have Q6_K v and down rows."""
    from torch2vk_amd.qwen3.config import QWEN3_0_6B
    from torch2vk_amd.qwen3.model import Qwen3Decoder
    from torch2vk_amd.qwen3.weights import matrix_shapes, synthetic_weights

    cfg = QWEN3_0_6B
    print(f"persistent 0.6B, 28 layers, {policy}: weights", flush=True)
    w = synthetic_weights(cfg, device=device, seed=0, std=0.02, norm_std=0.1, policy=policy)
    prompt = np.random.default_rng(0).integers(0, cfg.vocab, 128).tolist()
    dec = Qwen3Decoder(w, max_positions=256, max_new_tokens=40, persistent=True)
    assert dec.persistent
    dec.stop_on_eos = False
    toks = dec.generate(torch.tensor(prompt), 32, steps_per_graph=8, use_graph=True)
    assert int(dec.status.item()) == 0 and len(toks) == 32
    print(f"tokens {toks}", flush=True)
    # one more step's logits (RMSNorm -> bf16 -> LM-head GEMV over the persistent launch's h) against the
    # oracle's for the same token, position and KV history
    from oracle.qwen3_check import STEP_TOL_RMS, oracle_step_logits
    from tests.conftest import cosine

    pos, tok = int(dec.position.item()), int(dec.next_token.item())
    got = dec.step_logits(pos, token=tok).cpu().numpy()
    assert int(dec.status.item()) == 0
    shape = Qwen3Shape(hidden=cfg.hidden, layers=cfg.layers, heads=cfg.heads, kv_heads=cfg.kv_heads,
                       head_dim=cfg.head_dim, mlp=cfg.mlp, vocab=cfg.vocab, rope_theta=cfg.rope_theta)
    dense = dense_weights({k: v.cpu().numpy() for k, v in w.packed.items()}, w.types,
                          {k: v.cpu().numpy() for k, v in w.norms.items()}, matrix_shapes(cfg))
    ref = oracle_step_logits(shape, dense, dec.k_cache[:, :pos].cpu(), dec.v_cache[:, :pos].cpu(), tok, pos)
    rms = float(np.sqrt(np.mean(ref * ref)))
    err = float(np.abs(got - ref).max())
    print(f"step logits at pos {pos}: max-abs {err:.4f} (rms {rms:.3f}), cos {cosine(got, ref):.6f}", flush=True)
    # the per-step tolerance (3e-2 of the logits' rms; measured 1.5e-2 at 28 layers)
    assert err <= STEP_TOL_RMS * rms and cosine(got, ref) >= 0.9999
    stats = check_greedy_tokens(shape, dense, prompt, toks, kv_history=(dec.k_cache, dec.v_cache),
                                gpu_logits=decoder_step_logits(dec), label=f"0.6B 28 layers {policy}")
    print(stats, flush=True)


@pytest.mark.timeout(600)
def test_persistent_1_7b_full_depth_as_accurate_as_per_op(device):
    """The whole 28-layer Qwen3-1.7B decoder (hidden 2048, MLP 6144, vocab 151936) in the persistent kernel: a
    128-token random prompt fed one launch per position, then 32 greedy tokens in HIP graphs, status clear after
    all 160 launches.  Then one more step from that state, through the persistent launch and through the
    one-launch-per-op layers, each against the CPU oracle over the same KV history: the persistent kernel is no
    less accurate than the per-op path (bf16 activations carry 4-5 % of the logits' rms of rounding at this
    shape and depth in both, against 1.5 % at the 0.6B shape, so the 0.6B step bound does not transfer)."""
    from tests.conftest import cosine
    from oracle.qwen3_check import oracle_step_logits
    from torch2vk_amd.qwen3.config import QWEN3_1_7B
    from torch2vk_amd.qwen3.model import Qwen3Decoder
    from torch2vk_amd.qwen3.weights import matrix_shapes, synthetic_weights

    cfg = QWEN3_1_7B
    print("persistent 1.7B, 28 layers: weights", flush=True)
    w = synthetic_weights(cfg, device=device, seed=0, std=0.02, norm_std=0.1)
    prompt = np.random.default_rng(0).integers(0, cfg.vocab, 128).tolist()
    dec = Qwen3Decoder(w, max_positions=256, max_new_tokens=40, persistent=True)
    assert dec.persistent
    dec.stop_on_eos = False
    toks = dec.generate(torch.tensor(prompt), 32, steps_per_graph=8, use_graph=True)
    assert int(dec.status.item()) == 0 and len(toks) == 32
    print(f"tokens {toks}", flush=True)
    ref_dec = Qwen3Decoder(w, max_positions=256, max_new_tokens=40, persistent=False)
    ref_dec.k_cache.copy_(dec.k_cache)
    ref_dec.v_cache.copy_(dec.v_cache)
    pos, tok = int(dec.position.item()), int(dec.next_token.item())
    got = dec.step_logits(pos, token=tok).cpu().numpy()
    per_op = ref_dec.step_logits(pos, token=tok).cpu().numpy()
    assert int(dec.status.item()) == 0
    shape = Qwen3Shape(hidden=cfg.hidden, layers=cfg.layers, heads=cfg.heads, kv_heads=cfg.kv_heads,
                       head_dim=cfg.head_dim, mlp=cfg.mlp, vocab=cfg.vocab, rope_theta=cfg.rope_theta)
    dense = dense_weights({k: v.cpu().numpy() for k, v in w.packed.items()}, w.types,
                          {k: v.cpu().numpy() for k, v in w.norms.items()}, matrix_shapes(cfg))
    ref = oracle_step_logits(shape, dense, dec.k_cache[:, :pos].cpu(), dec.v_cache[:, :pos].cpu(), tok, pos)
    rms = float(np.sqrt(np.mean(ref * ref)))
    err, err_op = float(np.abs(got - ref).max()), float(np.abs(per_op - ref).max())
    print(f"step logits at pos {pos}: persistent max-abs {err:.4f}, per-op {err_op:.4f} (rms {rms:.3f}), "
          f"cos {cosine(got, ref):.6f}; argmax {got.argmax()} / {per_op.argmax()} / oracle {ref.argmax()}",
          flush=True)
    assert cosine(got, ref) >= 0.9999
    assert err <= 1.5 * err_op


# ------------------------------------------------------------------------------------------------------
# The Q4_K_M policy on the persistent kernel: with 2 layers, layer 1 is a more-bits layer (Q6_K v and down
# rows) and layer 0 is all Q4_K.


@pytest.fixture(scope="module", params=SHAPES)
def setup_km(device, request):
    from torch2vk_amd.qwen3.weights import synthetic_weights

    base = _base(request.param)
    cfg = replace(base, layers=2, vocab=4096, eos_token_ids=(4095,))
    w = synthetic_weights(cfg, device=device, seed=9, std=0.02, norm_std=0.1, policy="q4_k_m")
    assert (w.types["layers.0.v"], w.types["layers.0.down"]) == ("q4_k", "q4_k")
    assert (w.types["layers.1.v"], w.types["layers.1.down"]) == ("q6_k", "q6_k")
    shape = Qwen3Shape(hidden=cfg.hidden, layers=cfg.layers, heads=cfg.heads, kv_heads=cfg.kv_heads,
                       head_dim=cfg.head_dim, mlp=cfg.mlp, vocab=cfg.vocab, rope_theta=cfg.rope_theta)
    return cfg, w, shape


@pytest.mark.parametrize("layer,pos", [(1, 5), (1, 300), (0, 300)])
def test_persistent_q4_k_m_layer_matches_per_op(device, setup_km, layer, pos):
    """One Q4_K_M layer at one position: the q and k rows are bit-identical to the per-op Q4_K GEMV; a Q6_K
    v (layer 1) agrees with the per-op Q6_K GEMV to fp32 rounding (the persistent kernel runs x as fp16 with
    the offset 1056, the per-op kernel as bf16 with 160: both exact products of the same bf16 x); the
    attention output and h then as in test_persistent_layer_matches_per_op, through a Q6_K down at layer 1."""
    from torch2vk_amd.qwen3.model import Qwen3Decoder

    cfg, w, _ = setup_km
    print(f"persistent vs per-op, Q4_K_M layer {layer} at pos {pos}", flush=True)
    a = Qwen3Decoder(w, max_positions=512, max_new_tokens=4, persistent=True)
    b = Qwen3Decoder(w, max_positions=512, max_new_tokens=4, persistent=False)
    assert a.persistent and not b.persistent
    assert int(a.layer_table[1, 13]) == 3 and int(a.layer_table[0, 13]) == 0
    g = torch.Generator(device=device)
    g.manual_seed(11 + pos + layer)
    kc = torch.randn(a.k_cache.shape, generator=g, device=device).to(torch.bfloat16)
    vc = torch.randn(a.v_cache.shape, generator=g, device=device).to(torch.bfloat16)
    h0 = torch.randn(cfg.hidden, generator=g, device=device)
    for d in (a, b):
        d.k_cache.copy_(kc)
        d.v_cache.copy_(vc)
        d.h.copy_(h0)
        d.position.fill_(pos)
    a.layer_table = a.layer_table[layer:layer + 1].contiguous()
    a.run_decode_layers()
    b.run_decode_layer(layer)
    torch.cuda.synchronize()
    a.check_status()
    qkv = _ws_ll32(a, WS_QKV, cfg.q_dim + 2 * cfg.kv_dim)
    qk = cfg.q_dim + cfg.kv_dim
    torch.testing.assert_close(qkv[:qk], torch.cat([b.q, b.k]), rtol=0, atol=0)
    torch.testing.assert_close(a.k_cache[layer], b.k_cache[layer], rtol=0, atol=0)
    vmax = b.v.abs().max().item()
    if layer == 1:
        verr = (qkv[qk:] - b.v).abs().max().item()
        print(f"Q6_K v max-abs diff {verr:.3e} (max {vmax:.3e})", flush=True)
        assert verr <= 1e-5 * vmax
        # the new V row: one bf16 rounding of values that agree to ~1e-5, so at most one bf16 step apart
        vr_a, vr_b = a.v_cache[layer, pos].float(), b.v_cache[layer, pos].float()
        assert ((vr_a - vr_b).abs() <= 2 ** -7 * vr_b.abs() + 1e-30).all()
    else:
        torch.testing.assert_close(qkv[qk:], b.v, rtol=0, atol=0)
        torch.testing.assert_close(a.v_cache[layer], b.v_cache[layer], rtol=0, atol=0)
    attn = _ws_ll16(a, _ws_attn(cfg), cfg.q_dim).float()
    ref = b.attn.float()
    assert (attn - ref).abs().max().item() <= 2 ** -7 * ref.abs().max().item()
    herr = (a.h - b.h).abs().max().item()
    print(f"h max-abs diff {herr:.3e} (max {b.h.abs().max().item():.3e})", flush=True)
    assert herr <= 3e-3 * b.h.abs().max().item(), herr


def test_persistent_q4_k_m_decode_matches_oracle(device, setup_km):
    """Greedy decode with the persistent kernel on Q4_K_M weights (a Q4_K layer and a Q6_K v/down layer):
    prompt and 10 tokens through graph replay, every token against the CPU oracle."""
    from torch2vk_amd.qwen3.model import Qwen3Decoder
    from torch2vk_amd.qwen3.weights import matrix_shapes

    cfg, w, shape = setup_km
    dense = dense_weights({k: v.cpu().numpy() for k, v in w.packed.items()}, w.types,
                          {k: v.cpu().numpy() for k, v in w.norms.items()}, matrix_shapes(cfg))
    prompt = np.random.default_rng(4).integers(0, cfg.vocab, 5).tolist()
    dec = Qwen3Decoder(w, max_positions=128, max_new_tokens=16, persistent=True)
    assert dec.persistent
    dec.stop_on_eos = False
    toks = dec.generate(torch.tensor(prompt), 10, steps_per_graph=4, use_graph=True)
    dec.check_status()
    print(f"persistent Q4_K_M {cfg.name}-shape decode: {toks}", flush=True)
    print(check_greedy_tokens(shape, dense, prompt, toks, kv_history=(dec.k_cache, dec.v_cache),
                              gpu_logits=decoder_step_logits(dec), label=f"persistent Q4_K_M {cfg.name}"))
