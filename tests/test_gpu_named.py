"""The reference's unfused operators by name, and a whole prefill + greedy decode through the run_* dispatch
functions (src/models/optimized_qwen3/dispatch/*.py, src/models/optimized_qwen3/run.py:116-172,395-471) against
the CPU oracle."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import reference as R
from oracle.qwen3_check import check_greedy_tokens, decoder_step_logits, dense_weights
from oracle.reference import Qwen3Shape
from tests.conftest import assert_close

pytestmark = pytest.mark.gpu


def test_rope_table_closed_form(device):
    """cos / sin [B, T, D] = cos / sin of (start + t) theta^(-2 (d mod D/2) / D), fp32 against fp64, with the
    start position from an int and from a device counter; D 64 and 128."""
    from torch2vk_amd import variants as V
    from torch2vk_amd.runtime import RuntimeSession

    rt = RuntimeSession(device)
    for d, start, t_len in ((128, 4093, 7), (64, 0, 300)):
        cos = torch.zeros(2, t_len, d, device=device)
        sin = torch.zeros_like(cos)
        V.ROPE_TABLE_F32(rt, start_position=start, theta=1.0e6, cos=cos, sin=sin)
        pos = start + np.arange(t_len)
        inv = 1.0e6 ** (-(2.0 * (np.arange(d) % (d // 2))) / d)
        ang = pos[:, None] * inv[None, :]
        for got, ref in ((cos, np.cos(ang)), (sin, np.sin(ang))):
            g = got.cpu().numpy()
            assert np.array_equal(g[0], g[1])
            # fp32 angle: |pos * inv_freq| < 4e3 carries ~2.4e-4 of rounding
            assert np.abs(g[0] - ref).max() <= 5e-4, np.abs(g[0] - ref).max()
        dev_start = torch.tensor([start], dtype=torch.int32, device=device)
        cos2, sin2 = torch.zeros_like(cos), torch.zeros_like(sin)
        V.ROPE_TABLE_F32(rt, start_position=dev_start, theta=1.0e6, cos=cos2, sin=sin2)
        assert torch.equal(cos, cos2) and torch.equal(sin, sin2)


def test_norm_rope_from_table_equals_fused_prologue(device):
    """ROPE_TABLE_F32 + RMS_NORM_ROPE_TOKEN_F32 (q) / _TO_F16 (k) + TOKEN_MAJOR_*_CACHE_WRITE_*_PAIR give the
    chunk prologue's q and cache rows bit for bit (the same rope.h arithmetic, fp32 table); the transposed form
    is the same rows in [B, G, T, D]; both against the fp64 closed form."""
    from torch2vk_amd import kernels
    from torch2vk_amd import variants as V
    from torch2vk_amd.runtime import RuntimeSession

    rt = RuntimeSession(device)
    nh, nk, d, n, start, s_cap, theta = 8, 2, 128, 37, 100, 256, 1.0e6
    rng = np.random.default_rng(5)
    q = torch.from_numpy(rng.standard_normal((n, nh * d)).astype(np.float32)).to(device)
    k = torch.from_numpy(rng.standard_normal((n, nk * d)).astype(np.float32)).to(device)
    v = torch.from_numpy(rng.standard_normal((n, nk * d)).astype(np.float32)).to(device)
    qw = torch.from_numpy((1 + 0.1 * rng.standard_normal(d)).astype(np.float32)).to(device)
    kw = torch.from_numpy((1 + 0.1 * rng.standard_normal(d)).astype(np.float32)).to(device)
    kc = torch.zeros(s_cap, nk, d, dtype=torch.bfloat16, device=device)
    vc = torch.zeros_like(kc)
    qb = torch.empty(n, nh, d, dtype=torch.bfloat16, device=device)
    kernels.qk_norm_rope_cache(q, k, v, qb, kc, vc, start, q_norm_weight=qw, k_norm_weight=kw, theta=theta)

    cos = torch.zeros(1, n, d, device=device)
    sin = torch.zeros_like(cos)
    V.ROPE_TABLE_F32(rt, start_position=start, theta=theta, cos=cos, sin=sin)
    q_rot = torch.zeros(1, n, nh, d, dtype=torch.bfloat16, device=device)
    k_rot = torch.zeros(1, n, nk, d, dtype=torch.bfloat16, device=device)
    V.RMS_NORM_ROPE_TOKEN_F32(rt, x=q.view(1, n, nh, d), weight=qw, cos=cos, sin=sin, output=q_rot)
    V.RMS_NORM_ROPE_TOKEN_F32_TO_F16(rt, x=k.view(1, n, nk, d), weight=kw, cos=cos, sin=sin, output=k_rot)
    assert torch.equal(q_rot[0], qb)
    kc2 = torch.zeros(1, s_cap, nk, d, dtype=torch.bfloat16, device=device)
    vc2 = torch.zeros_like(kc2)
    other_k, other_v = torch.zeros_like(kc2), torch.zeros_like(kc2)
    pos = torch.arange(start, start + n, dtype=torch.int64, device=device)
    V.TOKEN_MAJOR_KV_CACHE_WRITE_F16_PAIR(rt, cache_a=kc2, cache_b=other_k, cache_position=pos, src=k_rot)
    V.TOKEN_MAJOR_VALUE_CACHE_WRITE_F32_TO_F16_PAIR(rt, cache_a=vc2, cache_b=other_v, cache_position=pos,
                                                    src=v.view(1, n, nk, d))
    assert torch.equal(kc2[0], kc) and torch.equal(vc2[0], vc)
    assert torch.equal(other_k, kc2) and torch.equal(other_v, vc2)
    # the transposed (decode) form and fp32 output
    q_t = torch.zeros(1, nh, n, d, device=device)
    V.RMS_NORM_ROPE_TRANSPOSE_F16(rt, x=q.view(1, n, nh, d), weight=qw, cos=cos, sin=sin, output=q_t)
    assert torch.equal(q_t[0].transpose(0, 1).to(torch.bfloat16), qb)
    c64, s64 = R.rope_cos_sin(start + np.arange(n), d, theta)
    ref = np.stack([R.qk_norm_rope(q.cpu().numpy().reshape(n, nh, d)[:, h], qw.cpu().numpy(), c64, s64)
                    for h in range(nh)], axis=1)
    assert_close(q_t[0].transpose(0, 1).cpu().numpy(), ref, max_abs=1e-4 * np.abs(ref).max(), min_cos=0.999999,
                 what="q norm + rope")


def test_kv_cache_write_positions(device):
    """Rows land at their cache_position in each cache (TRIPLE: three caches of different lengths); a position
    past a cache's length writes nothing there; fp32 sources are rounded to bf16 once."""
    from torch2vk_amd import variants as V
    from torch2vk_amd.runtime import RuntimeSession

    rt = RuntimeSession(device)
    b, t_len, h, d = 2, 5, 3, 128
    rng = np.random.default_rng(8)
    src = torch.from_numpy(rng.standard_normal((b, t_len, h, d)).astype(np.float32)).to(device)
    pos = torch.tensor([3, 0, 17, 9, 40], dtype=torch.int64, device=device)
    caches = [torch.full((b, s, h, d), 7.0, dtype=torch.bfloat16, device=device) for s in (20, 48, 10)]
    V.TOKEN_MAJOR_VALUE_CACHE_WRITE_F32_TO_F16_TRIPLE(rt, cache_a=caches[0], cache_b=caches[1], cache_c=caches[2],
                                                      cache_position=pos, src=src)
    sb = src.to(torch.bfloat16).cpu()
    for c in caches:
        ref = torch.full(c.shape, 7.0, dtype=torch.bfloat16)
        for ti, p in enumerate(pos.tolist()):
            if p < c.shape[1]:
                ref[:, p] = sb[:, ti]
        assert torch.equal(c.cpu(), ref)
    bf = src.to(torch.bfloat16)
    kc = [torch.zeros(b, 48, h, d, dtype=torch.bfloat16, device=device) for _ in range(2)]
    V.TOKEN_MAJOR_KV_CACHE_WRITE_F16_PAIR(rt, cache_a=kc[0], cache_b=kc[1], cache_position=pos, src=bf)
    for ti, p in enumerate(pos.tolist()):
        assert torch.equal(kc[0][:, p], bf[:, ti]) and torch.equal(kc[1][:, p], bf[:, ti])


def test_token_select_chunks_and_reduce(device):
    """QWEN3_TOKEN_SELECT_REDUCE_CHUNKS_F32 then QWEN3_TOKEN_SELECT_REDUCE_F32 over 5000 partials: the best
    score, ties to the lowest token id (ties planted within a chunk, across chunks, and in the last partial
    chunk); done set exactly when the winner is an EOS id."""
    from torch2vk_amd import variants as V
    from torch2vk_amd.runtime import RuntimeSession

    rt = RuntimeSession(device)
    g = 5000
    rng = np.random.default_rng(3)
    scores = rng.standard_normal(g).astype(np.float32)
    tokens = rng.permutation(100000)[:g].astype(np.int32)
    top = np.float32(9.0)
    for i in (17, 1500, 4999, 1023):  # tied maxima in chunks 0, 1 and 4
        scores[i] = top
    tokens[4999] = 5  # the lowest id among the tied ones, in the last, partial chunk
    for eos, want_done in ((np.array([5, 77]), 1), (np.array([6]), 0)):
        s_t = torch.from_numpy(scores).to(device)
        t_t = torch.from_numpy(tokens).to(device)
        cs = torch.zeros(5, device=device)
        ct = torch.zeros(5, dtype=torch.int32, device=device)
        V.QWEN3_TOKEN_SELECT_REDUCE_CHUNKS_F32(rt, scores=s_t, tokens=t_t, chunk_scores=cs, chunk_tokens=ct)
        for c in range(5):
            sl = slice(1024 * c, min(g, 1024 * (c + 1)))
            best = scores[sl].max()
            want_tok = tokens[sl][scores[sl] == best].min()
            assert cs[c].item() == best and ct[c].item() == want_tok, c
        nxt = torch.zeros(1, 1, dtype=torch.int64, device=device)
        done = torch.zeros(1, dtype=torch.int32, device=device)
        V.QWEN3_TOKEN_SELECT_REDUCE_F32(rt, partial_scores=cs, partial_tokens=ct,
                                        eos_token_ids=torch.from_numpy(eos).to(device), next_token=nxt, done=done)
        assert nxt.item() == 5 and done.item() == want_done
    with pytest.raises(ValueError, match="axis 0"):
        V.QWEN3_TOKEN_SELECT_REDUCE_CHUNKS_F32(rt, scores=s_t, tokens=t_t, chunk_scores=cs[:4], chunk_tokens=ct[:4])


def test_token_store_named(device):
    """QWEN3_TOKEN_STORE_EOS_F32 at a token index given as an int and as a device counter: the token lands at
    that index and the length follows; a selected EOS stops, and a stopped sequence stores nothing more."""
    from torch2vk_amd import variants as V
    from torch2vk_amd.runtime import RuntimeSession

    rt = RuntimeSession(device)
    gen = torch.full((1, 8), -1, dtype=torch.int64, device=device)
    length = torch.zeros(1, dtype=torch.int32, device=device)
    stopped = torch.zeros(1, dtype=torch.int32, device=device)
    done = torch.zeros(1, dtype=torch.int32, device=device)
    for idx, tok, is_eos in ((0, 11, 0), (torch.tensor([1], dtype=torch.int32, device=device), 12, 1), (2, 13, 0)):
        done.fill_(is_eos)
        V.QWEN3_TOKEN_STORE_EOS_F32(rt, next_token=torch.tensor([[tok]], device=device), token_index=idx, done=done,
                                    generated_tokens=gen, generated_length=length, stopped=stopped)
    assert gen.tolist()[0][:3] == [11, 12, -1] and length.item() == 2 and stopped.item() == 1


def _model(device, policy: str, seed: int):
    from torch2vk_amd.qwen3.config import Qwen3Config
    from torch2vk_amd.qwen3.weights import matrix_shapes, synthetic_weights

    cfg = Qwen3Config("named", hidden=1024, layers=3, heads=8, kv_heads=2, head_dim=128, mlp=1024, vocab=1024,
                      eos_token_ids=(1023,))
    w = synthetic_weights(cfg, device=device, seed=seed, std=0.05, norm_std=0.1, policy=policy)
    dense = dense_weights({k: v.cpu().numpy() for k, v in w.packed.items()}, w.types,
                          {k: v.cpu().numpy() for k, v in w.norms.items()}, matrix_shapes(cfg))
    shape = Qwen3Shape(hidden=cfg.hidden, layers=cfg.layers, heads=cfg.heads, kv_heads=cfg.kv_heads,
                       head_dim=cfg.head_dim, mlp=cfg.mlp, vocab=cfg.vocab, rope_theta=cfg.rope_theta)
    return cfg, w, dense, shape


@pytest.mark.parametrize("policy,prompt_len,chunk", [("uniform", 37, 16), ("q4_k_m", 41, 512)])
def test_named_prefill_and_decode_match_oracle(device, policy, prompt_len, chunk):
    """A prompt through run_prefill (a full chunk and the tail when the prompt is longer than ``chunk``, else the
    tail alone) and 10 greedy tokens through run_decode_step, every kernel launched by a named variant: the
    tokens against the CPU oracle (strict), the KV cache rows against the fused chunked prefill's, and the
    variants that ran against the reference's sequences."""
    from torch2vk_amd.qwen3 import dispatch as D
    from torch2vk_amd.qwen3.model import Qwen3Decoder
    from torch2vk_amd.runtime import RuntimeSession

    cfg, w, dense, shape = _model(device, policy, 71)
    prompt = np.random.default_rng(12).integers(0, cfg.vocab, prompt_len).tolist()
    dec = Qwen3Decoder(w, max_positions=96, max_new_tokens=16, persistent=False)
    dec.stop_on_eos = False
    rt = RuntimeSession(device, record=True)
    m = D.bind_model_tensors(dec)
    D.bind_prefill_tensors(torch.tensor(prompt), chunk=chunk)
    first = D.run_prefill(rt, rope_theta=cfg.rope_theta)
    prefill_h = m.prefill_last_output.view(-1).clone()
    names = [r.shader for r in rt.records]
    full = prompt_len > chunk
    assert names.count("rope_table_f32") == (2 if full else 1)
    assert names.count("token_major_kv_cache_write_f16_triple") == (cfg.layers if full else 0)
    assert names.count("token_major_kv_cache_write_f16_pair") == cfg.layers
    assert names.count("llama_flash_attn_f32_f16_f16") == cfg.layers * (2 if full else 1)
    assert names[-4:] == ["lm_head_q6_k_argmax_partial_f16" if policy == "q4_k_m" else
                          "lm_head_q4_k_argmax_partial_f16", "qwen3_token_select_reduce_chunks_f32",
                          "qwen3_token_select_reduce_f32", "qwen3_token_store_eos_f32"]
    if policy == "q4_k_m":
        assert "llama_matmul_q6_k_f32_m" in names and "linear_nobias_q6_k_matvec_f32" in names
    toks = [first]
    for step in range(9):
        toks.append(D.run_decode_step(rt, cache_position=prompt_len + step, rope_theta=cfg.rope_theta, step=step))
    torch.cuda.synchronize()
    assert dec.generated[:10].tolist() == toks and int(dec.length.item()) == 10
    print(f"named {policy}: {toks}", flush=True)
    # the named prefill's cache rows against the fused chunked prefill's (the same products, the q|k|v and
    # gate|up GEMMs run apart instead of stacked)
    ref = Qwen3Decoder(w, max_positions=96, max_new_tokens=16, persistent=False)
    ref.prefill_chunked(torch.tensor(prompt), chunk=chunk)
    torch.cuda.synchronize()
    for name in ("k_cache", "v_cache"):
        a = getattr(dec, name)[:, :prompt_len].float().cpu().numpy()
        b = getattr(ref, name)[:, :prompt_len].float().cpu().numpy()
        assert_close(a, b, max_abs=0.05 * np.abs(b).max(), min_cos=0.9999, what=name)
    stats = check_greedy_tokens(shape, dense, prompt, toks, kv_history=(dec.k_cache, dec.v_cache),
                                gpu_logits=decoder_step_logits(dec, prefill_h), label=f"named {policy}")
    print(stats, flush=True)
    assert math.isfinite(stats["min_margin"])


def test_exported_whole_prompt_names_match_oracle(device):
    """The exported path's run_embed_tokens, run_text_layer per layer and the final norm of every position
    (src/models/quantized_qwen3/export.py:254-315) over a 45-token prompt bound as one chunk, against the CPU
    oracle's causal pass over all positions (bf16 activations into the GEMMs and attention bound the error)."""
    from torch2vk_amd.qwen3 import dispatch as D
    from torch2vk_amd.qwen3.model import Qwen3Decoder
    from torch2vk_amd.runtime import RuntimeSession

    cfg, w, dense, shape = _model(device, "uniform", 73)
    prompt = np.random.default_rng(4).integers(0, cfg.vocab, 45).tolist()
    dec = Qwen3Decoder(w, max_positions=64, max_new_tokens=4, persistent=False)
    rt = RuntimeSession(device, record=True)
    D.bind_model_tensors(dec)
    D.bind_prefill_tensors(torch.tensor(prompt), chunk=len(prompt))
    D.run_embed_tokens(rt)
    for i in range(cfg.layers):
        D.run_text_layer(rt, i, rope_theta=cfg.rope_theta)
    out = torch.zeros(1, len(prompt), cfg.hidden, device=device)
    D.run_text_norm_all(rt, out)
    torch.cuda.synchronize()
    ref = R.Qwen3CpuModel(shape, dense, max_positions=64).forward(torch.tensor(prompt), 0, all_positions=True).numpy()
    got = out[0].cpu().numpy()
    print(f"exported names: max-abs {np.abs(got - ref).max():.3e} of max {np.abs(ref).max():.3e}", flush=True)
    assert_close(got, ref, max_abs=0.05 * float(np.abs(ref).max()), min_cos=0.999, what="normed hidden")
    names = [r.shader for r in rt.records]
    assert names[0] == "embedding_q4_k_act_f32" and names[-1] == "rms_norm_mul_f32"
