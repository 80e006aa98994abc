"""Several decode sequences in one persistent launch (t2h_qwen3_decode_layers_seqs, Qwen3DecoderGroup): 4
sequences of the Qwen3-0.6B shape on 64 blocks each, against the same decoders run one launch each and against
the CPU oracle."""

from __future__ import annotations

from dataclasses import replace

import numpy as np
import pytest
import torch

from oracle.qwen3_check import check_greedy_tokens, decoder_step_logits, dense_weights
from oracle.reference import Qwen3Shape

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def small_06b(device):
    from torch2vk_amd.qwen3.config import QWEN3_0_6B
    from torch2vk_amd.qwen3.weights import matrix_shapes, synthetic_weights

    cfg = replace(QWEN3_0_6B, layers=2, vocab=4096, eos_token_ids=(4095,))
    w = synthetic_weights(cfg, device=device, seed=12, std=0.02, norm_std=0.1)
    shape = Qwen3Shape(hidden=cfg.hidden, layers=cfg.layers, heads=cfg.heads, kv_heads=cfg.kv_heads,
                       head_dim=cfg.head_dim, mlp=cfg.mlp, vocab=cfg.vocab, rope_theta=cfg.rope_theta)
    dense = dense_weights({k: v.cpu().numpy() for k, v in w.packed.items()}, w.types,
                          {k: v.cpu().numpy() for k, v in w.norms.items()}, matrix_shapes(cfg))
    return cfg, w, shape, dense


def _decoders(w, n, max_positions):
    from torch2vk_amd.qwen3.model import Qwen3Decoder

    ds = [Qwen3Decoder(w, max_positions=max_positions, max_new_tokens=24, persistent=True) for _ in range(n)]
    for d in ds:
        d.stop_on_eos = False
    return ds


def test_group_short_prompts_equal_one_launch_each(device, small_06b):
    """Prompts of 4..13 tokens, then 12 tokens: every position stays under 256 keys, where one block per kv head
    covers the whole attention in both layouts, so the group's tokens, h and KV caches equal the single
    launches' bit for bit (the GEMV rows are the same dot products on other waves); graph replay included."""
    from torch2vk_amd.qwen3.model import Qwen3DecoderGroup

    cfg, w, _, _ = small_06b
    rng = np.random.default_rng(3)
    prompts = [rng.integers(0, cfg.vocab, n).tolist() for n in (4, 7, 13, 9)]
    single = _decoders(w, 4, 128)
    ref = [d.generate(torch.tensor(p), 12, steps_per_graph=4, use_graph=True) for d, p in zip(single, prompts)]
    group = _decoders(w, 4, 128)
    for d, p in zip(group, prompts):
        d.prefill(torch.tensor(p))
    got = Qwen3DecoderGroup(group).finish(12, steps_per_graph=4, use_graph=True)
    print(f"group {got}\nsingle {ref}", flush=True)
    assert got == ref
    for a, b, p in zip(group, single, prompts):
        n = len(p) + 12
        torch.testing.assert_close(a.h, b.h, rtol=0, atol=0)
        torch.testing.assert_close(a.k_cache[:, :n], b.k_cache[:, :n], rtol=0, atol=0)
        torch.testing.assert_close(a.v_cache[:, :n], b.v_cache[:, :n], rtol=0, atol=0)
        assert int(a.status.item()) == 0


def test_group_long_kv_matches_oracle(device, small_06b):
    """Four sequences from different N(0,1) KV caches of 600 .. 1500 positions (spans of 10 .. 24 positions per
    wave over 8 blocks per kv head, merged): a 2-token prompt each, then 6 tokens of group decode through graph
    replay; every sequence's tokens against the CPU oracle from its own cache, and the first group step's h
    against the single-launch decoder's within the summation-order tolerance of test_persistent_long_kv."""
    from torch2vk_amd.qwen3.model import Qwen3DecoderGroup

    cfg, w, shape, dense = small_06b
    starts = (600, 1023, 1300, 1500)
    group = _decoders(w, 4, 1536)
    g = torch.Generator(device=device)
    g.manual_seed(77)
    for d, st in zip(group, starts):
        d.k_cache[:, :st].normal_(generator=g)
        d.v_cache[:, :st].normal_(generator=g)
    prompts = [[11 + i, 2000 + i] for i in range(4)]
    for d, p, st in zip(group, prompts, starts):
        d.prefill(torch.tensor(p), start=st)
    # one group step against the same step on a single-launch copy of sequence 3
    from torch2vk_amd.qwen3.model import Qwen3Decoder
    solo = Qwen3Decoder(w, max_positions=1536, max_new_tokens=24, persistent=True)
    solo.stop_on_eos = False
    solo.k_cache.copy_(group[3].k_cache)
    solo.v_cache.copy_(group[3].v_cache)
    for t in ("h", "position", "next_token", "length", "generated", "done", "stopped"):
        getattr(solo, t).copy_(getattr(group[3], t))
    grp = Qwen3DecoderGroup(group)
    grp.decode_step()
    solo.decode_step()
    torch.cuda.synchronize()
    herr = (group[3].h - solo.h).abs().max().item()
    print(f"group vs single h after one step at KV {starts[3] + 2}: {herr:.3e}", flush=True)
    assert herr <= 3e-3 * solo.h.abs().max().item()
    grp.run_steps(5, steps_per_graph=4, use_graph=True)
    for d, p, st in zip(group, prompts, starts):
        d.check_status()
        toks = d.generated[:int(d.length.item())].tolist()
        assert len(toks) == 7
        kv = (d.k_cache[:, :st].cpu(), d.v_cache[:, :st].cpu())
        print(f"start {st}: {toks}", flush=True)
        print(check_greedy_tokens(shape, dense, p, toks, start=st, kv_init=kv, kv_history=(d.k_cache, d.v_cache),
                                  gpu_logits=decoder_step_logits(d), label=f"group from KV {st}"), flush=True)


def test_group_rejects_bad_arguments(device, small_06b):
    from torch2vk_amd import kernels
    from torch2vk_amd.qwen3.model import Qwen3DecoderGroup

    cfg, w, _, _ = small_06b
    ds = _decoders(w, 4, 128)
    with pytest.raises(ValueError, match="runs"):
        Qwen3DecoderGroup(ds[:3])
    args = dict(hidden=cfg.hidden, mlp=cfg.mlp, nh=cfg.heads, nk=cfg.kv_heads, d=cfg.head_dim, s_cap=128)
    with pytest.raises(ValueError, match="own workspace"):
        kernels.decode_layers_seqs([d.layer_table for d in ds], [d.h for d in ds], [d.position for d in ds],
                                   [ds[0].layers_ws] * 4, [d.status for d in ds], **args)
    # the 8B shape is not built for 4 sequences: the library refuses before launching
    with pytest.raises(RuntimeError):
        kernels.decode_layers_seqs([d.layer_table for d in ds], [d.h for d in ds], [d.position for d in ds],
                                   [d.layers_ws for d in ds], [d.status for d in ds],
                                   **{**args, "hidden": 4096, "mlp": 12288, "nh": 32})
    # KV capacity over 2048 positions is refused for 4 sequences
    with pytest.raises(RuntimeError):
        kernels.decode_layers_seqs([d.layer_table for d in ds], [d.h for d in ds], [d.position for d in ds],
                                   [d.layers_ws for d in ds], [d.status for d in ds], **{**args, "s_cap": 4096})


def test_group_batched_prefill_matches_each_prefill(device, small_06b):
    """Four equal-length prompts of input embeddings prefilled as one batch (Qwen3DecoderGroup.create's
    layer-major caches) against each decoder's own chunked prefill, chunks of 64 over 150 positions: the same
    products, summed in another order where the single prefill's small GEMMs split K, so the caches and the
    last hidden state agree to bf16 rounding; the first tokens and 6 more of group decode against the oracle."""
    from torch2vk_amd.qwen3.model import Qwen3DecoderGroup

    cfg, w, shape, dense = small_06b
    group = Qwen3DecoderGroup.create(w, 4, max_positions=256, max_new_tokens=24, device=device)
    for d in group.decoders:
        d.stop_on_eos = False
    single = _decoders(w, 4, 256)
    rng = np.random.default_rng(9)
    prompts = [rng.integers(0, cfg.vocab, 150).tolist() for _ in range(4)]
    embs = [group.decoders[0].embed_tokens(torch.tensor(p, device=device)) for p in prompts]
    group.prefill_chunked(embs, chunk=64)
    prefill_h = [d.h.clone() for d in group.decoders]  # step 0's tokens come from these rows
    for d, e in zip(single, embs):
        d.prefill_chunked(embeds=e, chunk=64)
    torch.cuda.synchronize()
    for a, b in zip(group.decoders, single):
        for ca, cb in ((a.k_cache[:, :150], b.k_cache[:, :150]), (a.v_cache[:, :150], b.v_cache[:, :150])):
            # layer 0 sees the same inputs: its rows agree to one bf16 rounding of a reordered fp32 sum
            d0 = (ca[0].float() - cb[0].float()).abs()
            assert (d0 <= 2 ** -7 * cb[0].float().abs() + 1e-3).all(), d0.max().item()
            # layer 1 inherits layer 0's bf16-level differences through attention, o_proj and the MLP
            d1 = (ca[1].float() - cb[1].float()).abs().max().item()
            assert d1 <= 1e-2 * cb[1].float().abs().max().item(), d1
        assert int(a.position.item()) == int(b.position.item()) == 150
    toks = group.finish(7, steps_per_graph=4, use_graph=True)
    for b, (d, p, tk) in enumerate(zip(group.decoders, prompts, toks)):
        assert len(tk) == 7
        print(check_greedy_tokens(shape, dense, p, tk, kv_history=(d.k_cache, d.v_cache),
                                  gpu_logits=decoder_step_logits(d, prefill_h[b]), label=f"batched prefill {b}"),
              flush=True)


def test_group_q4_k_m_equals_one_launch_each(device):
    """Q4_K_M weights (layer 1 of 2 with Q6_K v and down rows) in the 4-sequence launch: at 64 blocks per
    sequence a Q6_K v lands in each wave's second Q|K|V slot and the Q6_K down units spread over the blocks;
    short prompts keep every position under 256 keys, so tokens, h and caches equal the single launches'."""
    from torch2vk_amd.qwen3.config import QWEN3_0_6B
    from torch2vk_amd.qwen3.model import Qwen3DecoderGroup
    from torch2vk_amd.qwen3.weights import synthetic_weights

    cfg = replace(QWEN3_0_6B, layers=2, vocab=4096, eos_token_ids=(4095,))
    w = synthetic_weights(cfg, device=device, seed=21, std=0.02, norm_std=0.1, policy="q4_k_m")
    assert (w.types["layers.1.v"], w.types["layers.1.down"]) == ("q6_k", "q6_k")
    rng = np.random.default_rng(8)
    prompts = [rng.integers(0, cfg.vocab, n).tolist() for n in (6, 3, 10, 8)]
    single = _decoders(w, 4, 128)
    ref = [d.generate(torch.tensor(p), 10, steps_per_graph=4, use_graph=True) for d, p in zip(single, prompts)]
    group = _decoders(w, 4, 128)
    for d, p in zip(group, prompts):
        d.prefill(torch.tensor(p))
    got = Qwen3DecoderGroup(group).finish(10, steps_per_graph=4, use_graph=True)
    print(f"group {got}\nsingle {ref}", flush=True)
    assert got == ref
    for a, b in zip(group, single):
        torch.testing.assert_close(a.h, b.h, rtol=0, atol=0)
        torch.testing.assert_close(a.v_cache, b.v_cache, rtol=0, atol=0)


def test_group_traced_launch_equals_untraced(device, small_06b):
    """The timeline instantiation of the 4-sequence launch (t2h_qwen3_decode_layers_seqs_traced) computes the same
    bits as the plain one and stamps every sequence's 64 blocks in every phase it runs."""
    from torch2vk_amd import kernels
    from torch2vk_amd.qwen3.model import Qwen3DecoderGroup

    cfg, w, _, _ = small_06b
    a, b = _decoders(w, 4, 512), _decoders(w, 4, 512)
    g = torch.Generator(device=device)
    g.manual_seed(21)
    for i, (da, db) in enumerate(zip(a, b)):
        kc = torch.randn(da.k_cache.shape, generator=g, device=device).to(torch.bfloat16)
        vc = torch.randn(da.v_cache.shape, generator=g, device=device).to(torch.bfloat16)
        h0 = torch.randn(cfg.hidden, generator=g, device=device)
        for d in (da, db):
            d.k_cache.copy_(kc)
            d.v_cache.copy_(vc)
            d.h.copy_(h0)
            d.position.fill_(100 + 100 * i)  # one sequence past 256 keys: the merge phase runs
    trace = kernels.decode_layers_trace(cfg.layers, device)
    Qwen3DecoderGroup(a).run_decode_layers(trace=trace)
    Qwen3DecoderGroup(b).run_decode_layers()
    torch.cuda.synchronize()
    for da, db in zip(a, b):
        da.check_status()
        db.check_status()
        torch.testing.assert_close(da.h, db.h, rtol=0, atol=0)
        torch.testing.assert_close(da.k_cache, db.k_cache, rtol=0, atol=0)
    tr = trace.cpu()
    for ph in (0, 3, 4, 5):  # qkv, o, gate|up, down: every block of every sequence
        assert (tr[:, ph, :, 3] != 0).all(), ph
    assert (tr[:, 2, 192:192 + cfg.heads, 3] != 0).all()  # sequence 3 (400 positions) merged its q heads
