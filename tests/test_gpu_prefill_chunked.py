"""GPU parity of the chunked matrix-core prefill: the chunk prologue kernel against the decode prologue
(bit-exact cache rows) and the numpy oracle, and whole prompts prefilled in chunks against the CPU oracle
decoder (greedy tokens, exact) and against the token-by-token prefill's KV cache."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import reference as R
from oracle.qwen3_check import check_greedy_tokens, decoder_step_logits, dense_weights
from oracle.reference import Qwen3Shape
from tests.conftest import assert_close

pytestmark = pytest.mark.gpu


def test_chunk_prologue_matches_decode_prologue_and_oracle(device):
    from torch2vk_amd import kernels

    nh, nk, d, n, start, s_cap, theta = 8, 2, 128, 37, 100, 256, 1e6
    rng = np.random.default_rng(0)
    q = rng.standard_normal((n, nh * d)).astype(np.float32)
    k = rng.standard_normal((n, nk * d)).astype(np.float32) * 3
    v = rng.standard_normal((n, nk * d)).astype(np.float32)
    qw = (1 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    kw = (1 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    qkv = torch.from_numpy(np.concatenate([q, k, v], axis=1)).to(device)
    kc = torch.zeros(s_cap, nk, d, dtype=torch.bfloat16, device=device)
    vc = torch.zeros_like(kc)
    qb = torch.empty(n, nh, d, dtype=torch.bfloat16, device=device)
    qwt, kwt = torch.from_numpy(qw).to(device), torch.from_numpy(kw).to(device)
    kernels.qk_norm_rope_cache(qkv[:, :nh * d], qkv[:, nh * d:(nh + nk) * d], qkv[:, (nh + nk) * d:], qb, kc, vc,
                               start, q_norm_weight=qwt, k_norm_weight=kwt, theta=theta)
    # numpy oracle
    cos, sin = R.rope_cos_sin(np.arange(start, start + n), d, theta)
    q_ref = R.qk_norm_rope(q.reshape(n, nh, d), qw, cos[:, None, :], sin[:, None, :])
    k_ref = R.qk_norm_rope(k.reshape(n, nk, d), kw, cos[:, None, :], sin[:, None, :])
    assert_close(qb.float().cpu().numpy(), q_ref, max_abs=3e-2, min_cos=0.9999, what="q")
    assert_close(kc[start:start + n].float().cpu().numpy(), k_ref, max_abs=1e-1, min_cos=0.9999, what="k")
    assert torch.equal(vc[start:start + n].cpu(), torch.from_numpy(v.reshape(n, nk, d)).to(torch.bfloat16))
    assert not kc[:start].any() and not kc[start + n:].any()
    # the decode prologue writes the same bits for the same token at the same position
    kd = torch.zeros_like(kc)
    vd = torch.zeros_like(kc)
    ws = kernels.attn_decode_workspace(nh, nk, d, s_cap, device)
    out = torch.empty(nh * d, dtype=torch.bfloat16, device=device)
    for t in (0, 17, n - 1):
        pos = torch.tensor([start + t], dtype=torch.int32, device=device)
        kernels.attn_decode(qkv[t, :nh * d].contiguous(), qkv[t, nh * d:(nh + nk) * d].contiguous(),
                            qkv[t, (nh + nk) * d:].contiguous(), kd, vd, out, pos, ws, q_norm_weight=qwt,
                            k_norm_weight=kwt, theta=theta)
        assert torch.equal(kd[start + t], kc[start + t]), t
        assert torch.equal(vd[start + t], vc[start + t]), t


@pytest.mark.parametrize("nh,nk", [(8, 2), (32, 8)])
def test_chunk_prologue_batched_equals_per_sequence(device, nh, nk):
    """n_seq sequences in one launch (q|k|v rows sequence after sequence, one cache per sequence) write the
    same bits as one call per sequence."""
    from torch2vk_amd import kernels

    n_seq, n, d, start, s_cap, theta = 3, 37, 128, 100, 256, 1e6
    rng = np.random.default_rng(nh)
    qkv = torch.from_numpy(rng.standard_normal((n_seq * n, (nh + 2 * nk) * d)).astype(np.float32)).to(device)
    qw = torch.from_numpy((1 + 0.1 * rng.standard_normal(d)).astype(np.float32)).to(device)
    kw = torch.from_numpy((1 + 0.1 * rng.standard_normal(d)).astype(np.float32)).to(device)
    q, k, v = qkv[:, :nh * d], qkv[:, nh * d:(nh + nk) * d], qkv[:, (nh + nk) * d:]
    kc = torch.zeros(n_seq, s_cap, nk, d, dtype=torch.bfloat16, device=device)
    vc = torch.zeros_like(kc)
    qb = torch.empty(n_seq * n, nh, d, dtype=torch.bfloat16, device=device)
    kernels.qk_norm_rope_cache(q, k, v, qb, kc, vc, start, q_norm_weight=qw, k_norm_weight=kw, theta=theta)
    kc1, vc1 = torch.zeros_like(kc), torch.zeros_like(kc)
    qb1 = torch.empty_like(qb)
    for sq in range(n_seq):
        r = slice(sq * n, (sq + 1) * n)
        kernels.qk_norm_rope_cache(q[r], k[r], v[r], qb1[r], kc1[sq], vc1[sq], start, q_norm_weight=qw,
                                   k_norm_weight=kw, theta=theta)
    assert torch.equal(qb, qb1)
    assert torch.equal(kc, kc1) and torch.equal(vc, vc1)
    assert not kc[:, :start].any() and not kc[:, start + n:].any()


def _setup(cfg, device, seed, std, policy):
    from torch2vk_amd.qwen3.weights import matrix_shapes, synthetic_weights

    w = synthetic_weights(cfg, device=device, seed=seed, std=std, norm_std=0.1, policy=policy)
    dense = dense_weights({k: v.cpu().numpy() for k, v in w.packed.items()}, w.types,
                          {k: v.cpu().numpy() for k, v in w.norms.items()}, matrix_shapes(cfg))
    shape = Qwen3Shape(hidden=cfg.hidden, layers=cfg.layers, heads=cfg.heads, kv_heads=cfg.kv_heads,
                       head_dim=cfg.head_dim, mlp=cfg.mlp, vocab=cfg.vocab, rope_theta=cfg.rope_theta)
    return w, dense, shape


@pytest.mark.parametrize("policy,chunk", [("uniform", 16), ("q4_k_m", 5), ("uniform", 4096)])
def test_chunked_prefill_decode_matches_oracle(device, policy, chunk):
    from torch2vk_amd.qwen3.config import Qwen3Config
    from torch2vk_amd.qwen3.model import Qwen3Decoder

    cfg = Qwen3Config("tiny-p", hidden=1024, layers=4, heads=8, kv_heads=2, head_dim=128, mlp=1024, vocab=1024,
                      eos_token_ids=(1023,))
    w, dense, shape = _setup(cfg, device, seed=31, std=0.05, policy=policy)
    prompt = np.random.default_rng(2).integers(0, cfg.vocab, 37).tolist()
    dec = Qwen3Decoder(w, max_positions=96, max_new_tokens=16)
    dec.stop_on_eos = False
    dec.prefill_chunked(torch.tensor(prompt), chunk=chunk)
    prefill_h = dec.h.clone()  # the first token is selected from this row
    dec.run_steps(9, steps_per_graph=4)
    toks = dec.generated[:int(dec.length.item())].tolist()
    print(f"chunked prefill {policy} chunk={chunk}: {toks}", flush=True)
    assert len(toks) == 10
    print(check_greedy_tokens(shape, dense, prompt, toks, kv_history=(dec.k_cache, dec.v_cache),
                              gpu_logits=decoder_step_logits(dec, prefill_h), label=f"chunked {policy} {chunk}"))


def test_chunked_prefill_cache_matches_token_prefill(device):
    from torch2vk_amd.qwen3.config import Qwen3Config
    from torch2vk_amd.qwen3.model import Qwen3Decoder

    cfg = Qwen3Config("tiny-p", hidden=1024, layers=3, heads=8, kv_heads=2, head_dim=128, mlp=1024, vocab=1024,
                      eos_token_ids=(1023,))
    w, _, _ = _setup(cfg, device, seed=41, std=0.05, policy="uniform")
    prompt = torch.tensor(np.random.default_rng(3).integers(0, cfg.vocab, 50).tolist())
    a = Qwen3Decoder(w, max_positions=64, max_new_tokens=4)
    b = Qwen3Decoder(w, max_positions=64, max_new_tokens=4)
    a.prefill(prompt)
    b.prefill_chunked(prompt, chunk=20)
    torch.cuda.synchronize()
    n = prompt.numel()
    for name in ("k_cache", "v_cache"):
        ca = getattr(a, name)[:, :n].float().cpu().numpy()
        cb = getattr(b, name)[:, :n].float().cpu().numpy()
        assert_close(cb, ca, max_abs=0.1 * np.abs(ca).max(), min_cos=0.999, what=name)
        assert not getattr(b, name)[:, n:].any()
    assert int(a.position.item()) == int(b.position.item()) == n
    assert int(a.length.item()) == int(b.length.item()) == 1


def test_chunked_prefill_from_embeds_equals_ids(device):
    """A prompt given as its own embedding rows prefills exactly like the ids (same kernels, same bits)."""
    from torch2vk_amd.qwen3.config import Qwen3Config
    from torch2vk_amd.qwen3.model import Qwen3Decoder

    cfg = Qwen3Config("tiny-p", hidden=1024, layers=2, heads=8, kv_heads=2, head_dim=128, mlp=1024, vocab=1024,
                      eos_token_ids=(1023,))
    w, _, _ = _setup(cfg, device, seed=51, std=0.05, policy="qwen3_asr")
    prompt = torch.tensor(np.random.default_rng(4).integers(0, cfg.vocab, 23).tolist(), device=device)
    a = Qwen3Decoder(w, max_positions=48, max_new_tokens=8)
    b = Qwen3Decoder(w, max_positions=48, max_new_tokens=8)
    a.stop_on_eos = b.stop_on_eos = False
    ta = a.generate(prompt, 6, prefill_chunk=8)
    tb = b.generate_from_embeds(b.embed_tokens(prompt), 6, prefill_chunk=8)
    assert ta == tb
    assert torch.equal(a.k_cache, b.k_cache)


@pytest.mark.parametrize("policy", ["uniform", "q4_k_m"])
def test_forward_masked_matches_oracle(device, policy):
    """OmniVoice's LLM pass: every layer over a whole sequence under an additive mask (padded keys, a
    bidirectional block and a hole), then the final norm of every position, against the CPU oracle's masked
    pass on the same dequantized weights.  bf16 activations into the GEMMs and attention bound the error."""
    from torch2vk_amd.qwen3.config import Qwen3Config
    from torch2vk_amd.qwen3.model import Qwen3Decoder

    cfg = Qwen3Config("tiny-p", hidden=1024, layers=2, heads=8, kv_heads=2, head_dim=128, mlp=1024, vocab=1024,
                      eos_token_ids=(1023,))
    w, dense, shape = _setup(cfg, device, seed=61, std=0.05, policy=policy)
    t = 45
    ids = torch.tensor(np.random.default_rng(6).integers(0, cfg.vocab, t).tolist(), device=device)
    dec = Qwen3Decoder(w, max_positions=64, max_new_tokens=4)
    emb = dec.embed_tokens(ids)
    mask = torch.zeros(t, t)
    mask[:, 38:] = float("-inf")        # padded keys hidden from every query ...
    mask[38:, 38:] = 0.0                # ... except from the padded queries
    mask[:20, 20:38] = float("-inf")    # the first 20 positions attend only among themselves
    mask[3, 7] = float("-inf")          # and one hole
    out = dec.forward_masked(emb, mask.to(device))
    torch.cuda.synchronize()
    ref = R.Qwen3CpuModel(shape, dense, max_positions=64).forward(None, 0, embeds=emb.cpu(), mask=mask,
                                                                  all_positions=True)
    got, ref = out.cpu().numpy(), ref.numpy()
    print(f"forward_masked {policy}: max-abs {np.abs(got - ref).max():.3e}, max |ref| {np.abs(ref).max():.3e}",
          flush=True)
    assert_close(got, ref, max_abs=0.05 * float(np.abs(ref).max()), min_cos=0.999, what="final hidden")
    for row in (0, 19, 20, 37, 44):
        assert_close(got[row], ref[row], max_abs=0.05 * float(np.abs(ref).max()), min_cos=0.999, what=f"row {row}")


def test_graphed_prefill_equals_eager_prefill(device):
    """prefill_graphed replays one captured prefill: three prompts of one length, with eager decode steps
    between the replays, each give prefill_chunked's KV cache, token and counters bit for bit."""
    from torch2vk_amd.qwen3.config import Qwen3Config
    from torch2vk_amd.qwen3.model import Qwen3Decoder

    cfg = Qwen3Config("tiny-p", hidden=1024, layers=3, heads=8, kv_heads=2, head_dim=128, mlp=1024, vocab=1024,
                      eos_token_ids=(1023,))
    w, _, _ = _setup(cfg, device, seed=61, std=0.05, policy="uniform")
    a = Qwen3Decoder(w, max_positions=80, max_new_tokens=8)
    b = Qwen3Decoder(w, max_positions=80, max_new_tokens=8)
    a.stop_on_eos = b.stop_on_eos = False
    rng = np.random.default_rng(7)
    for rep in range(3):
        prompt = torch.tensor(rng.integers(0, cfg.vocab, 50).tolist(), device=device)
        a.prefill_chunked(prompt, chunk=20)
        b.prefill_graphed(prompt, chunk=20)
        torch.cuda.synchronize()
        for name in ("k_cache", "v_cache", "next_token", "position", "length", "generated", "h"):
            assert torch.equal(getattr(a, name), getattr(b, name)), (rep, name)
        a.run_steps(3, use_graph=False)
        b.run_steps(3, use_graph=False)
        assert torch.equal(a.generated, b.generated), rep
    assert len(b._prefill_graphs) == 1
