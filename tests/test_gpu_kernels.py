"""GPU parity of the libt2h kernels against the CPU oracle (calls go through the C ABI)."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import oracle
from oracle import reference as R
from tests.conftest import assert_close

pytestmark = pytest.mark.gpu


def _special_rows(k: int, rng: np.random.Generator) -> np.ndarray:
    """Rows exercising the quantizers' special branches."""
    rows = [
        np.zeros(k),                                   # all zero: d = dmin = 0
        np.full(k, 0.37),                              # constant positive: max == min branch
        np.full(k, -1.25),                             # constant negative
        np.abs(rng.standard_normal(k)),                # non-negative: min clamps to 0
        -np.abs(rng.standard_normal(k)),               # non-positive
        rng.standard_normal(k) * 1e-20,                # tiny (fp16 subnormal / zero scales)
        rng.standard_normal(k) * 3e3,                  # large
        np.where(np.arange(k) % 32 == 5, 7.0, 0.0),    # one spike per 32
        rng.standard_normal(k) * np.repeat(10.0 ** rng.uniform(-4, 1, k // 16), 16),  # mixed block scales
    ]
    return np.stack(rows).astype(np.float32)


@pytest.mark.parametrize("wtype,k", [("q4_k", 1024), ("q4_k", 4096), ("q6_k", 1024), ("q6_k", 4096),
                                     ("q8_0", 1024), ("q8_0", 96)])
def test_quantizer_bit_exact(device, wtype, k):
    rng = np.random.default_rng(1234 + k)
    x = np.concatenate([(rng.standard_normal((120, k)) * 0.02).astype(np.float32),
                        (rng.standard_normal((4, k)) * 5).astype(np.float32),
                        _special_rows(k, rng)])
    print(f"quantizer {wtype} K={k} rows={x.shape[0]}", flush=True)
    from torch2vk_amd import kernels

    got = kernels.quantize(torch.from_numpy(x).to(device), wtype).cpu().numpy()
    ref = getattr(oracle, f"quantize_{wtype}")(x)
    assert got.shape == ref.shape
    bad = np.argwhere(got != ref)
    assert bad.size == 0, f"{len(bad)} bytes differ, first at {bad[:4].tolist()}"


@pytest.mark.parametrize("wtype", ["q4_k", "q6_k", "q8_0"])
def test_dequantize_matches_oracle(device, wtype):
    rng = np.random.default_rng(7)
    k = 512
    x = (rng.standard_normal((64, k)) * 0.05).astype(np.float32)
    packed = getattr(oracle, f"quantize_{wtype}")(x)
    from torch2vk_amd import kernels

    got = kernels.dequantize(torch.from_numpy(packed).to(device), wtype, k).cpu().numpy()
    ref = getattr(oracle, f"dequant_{wtype}")(packed, k)
    np.testing.assert_array_equal(got, ref)


def _q4_problem(n, k, seed):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    packed = oracle.quantize_q4_k(w)
    wd = oracle.dequant_q4_k(packed, k)
    return rng, packed, wd


@pytest.mark.parametrize("n,k", [(64, 256), (96, 768), (2048, 1024), (3072, 1024), (256, 3072), (512, 4096),
                                 (128, 12288), (40, 8192)])
def test_q4k_matvec(device, n, k):
    from torch2vk_amd import kernels

    print(f"q4k_matvec N={n} K={k}", flush=True)
    rng, packed, wd = _q4_problem(n, k, n + k)
    x = R.bf16_round(rng.standard_normal(k).astype(np.float32))
    ref = R.gemv_ref(x, wd)
    wt = torch.from_numpy(packed).to(device)
    xt = torch.from_numpy(x).to(device).to(torch.bfloat16)
    got = kernels.q4k_matvec(xt, wt).cpu().numpy()
    assert_close(got, ref, max_abs=2e-4 * np.abs(ref).max() + 1e-6, min_cos=0.99999, what="f32 out")
    # residual epilogue, in place
    res = rng.standard_normal(n).astype(np.float32)
    rt = torch.from_numpy(res).to(device)
    kernels.q4k_matvec(xt, wt, out=rt, residual=rt)
    assert_close(rt.cpu().numpy(), ref + res, max_abs=2e-4 * np.abs(ref).max() + 1e-5, min_cos=0.99999,
                 what="residual")
    # bf16 out
    got16 = kernels.q4k_matvec(xt, wt, out_dtype=torch.bfloat16).float().cpu().numpy()
    assert_close(got16, ref, max_abs=1e-2 * np.abs(ref).max() + 1e-6, min_cos=0.9999, what="bf16 out")


def test_q4k_matvec_multi_rows(device):
    """M > 1 tokens (the reference matvec accepts M <= 8)."""
    from torch2vk_amd import kernels

    n, k, m = 256, 2048, 3
    rng, packed, wd = _q4_problem(n, k, 5)
    x = R.bf16_round(rng.standard_normal((m, k)).astype(np.float32))
    ref = R.gemv_ref(x, wd)
    got = kernels.q4k_matvec(torch.from_numpy(x).to(device).to(torch.bfloat16),
                             torch.from_numpy(packed).to(device)).cpu().numpy()
    assert_close(got, ref, max_abs=2e-4 * np.abs(ref).max(), min_cos=0.99999, what="M=3")


@pytest.mark.parametrize("k,ns", [(1024, (2048, 1024, 1024)), (4096, (512, 128, 128)), (3072, (96, 32))])
def test_q4k_multi_rmsnorm_prologue(device, k, ns):
    from torch2vk_amd import kernels

    print(f"q4k multi K={k} parts={ns}", flush=True)
    rng = np.random.default_rng(k)
    h = (rng.standard_normal(k) * 3).astype(np.float32)
    nw = (1 + 0.1 * rng.standard_normal(k)).astype(np.float32)
    xn = R.bf16_round(R.rms_norm(h, nw).astype(np.float32))
    packs, outs, refs = [], [], []
    for i, n in enumerate(ns):
        w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
        p = oracle.quantize_q4_k(w)
        packs.append(torch.from_numpy(p).to(device))
        outs.append(torch.empty(n, dtype=torch.float32, device=device))
        refs.append(R.gemv_ref(xn, oracle.dequant_q4_k(p, k)))
    kernels.q4k_matvec_multi(torch.from_numpy(h).to(device), packs, outs,
                             norm_weight=torch.from_numpy(nw).to(device))
    for i, (o, r) in enumerate(zip(outs, refs)):
        # x is rounded to bf16 after the norm; one-ulp flips of that rounding bound the error
        assert_close(o.cpu().numpy(), r, max_abs=5e-3 * np.abs(r).max(), min_cos=0.9999, what=f"part {i}")


@pytest.mark.parametrize("k,n", [(1024, 3072), (4096, 1024), (3072, 256)])
def test_q4k_rmsnorm_swiglu(device, k, n):
    from torch2vk_amd import kernels

    rng = np.random.default_rng(n)
    h = (rng.standard_normal(k) * 2).astype(np.float32)
    nw = (1 + 0.1 * rng.standard_normal(k)).astype(np.float32)
    wg = oracle.quantize_q4_k((rng.standard_normal((n, k)) * 0.05).astype(np.float32))
    wu = oracle.quantize_q4_k((rng.standard_normal((n, k)) * 0.05).astype(np.float32))
    xn = R.bf16_round(R.rms_norm(h, nw).astype(np.float32))
    ref = R.silu_mul(R.gemv_ref(xn, oracle.dequant_q4_k(wg, k)), R.gemv_ref(xn, oracle.dequant_q4_k(wu, k)))
    out = torch.empty(n, dtype=torch.bfloat16, device=device)
    kernels.q4k_rmsnorm_swiglu(torch.from_numpy(h).to(device), torch.from_numpy(nw).to(device),
                               torch.from_numpy(wg).to(device), torch.from_numpy(wu).to(device), out)
    assert_close(out.float().cpu().numpy(), ref, max_abs=2e-2 * np.abs(ref).max(), min_cos=0.9995, what="swiglu")



def _best_pair(scores: torch.Tensor, tokens: torch.Tensor) -> tuple[int, int]:
    """The selected (score bits, token) of a partial set: highest score, ties to the lower token id."""
    sc = scores.cpu().numpy().astype(np.float64)
    tk = tokens.cpu().numpy().view(np.uint32).astype(np.int64)
    i = int(np.lexsort((tk, -sc))[0])
    return int(scores.cpu().numpy().view(np.uint32)[i]), int(tk[i])


@pytest.mark.parametrize("k,n,g", [(1024, 5000, 64), (1024, 151936, 512), (4096, 20000, 96), (1024, 5000, 1024)])
def test_lm_head_seqs_equals_each_sequence(device, k, n, g):
    """The LM head of 1..4 sequences in one launch: every sequence's best (score, token) pair over its
    partials is bit-identical to its own single-sequence launch's (one sequence: every partial is), including
    a tie between two equal rows (the lower id)."""
    from torch2vk_amd import kernels

    rng = np.random.default_rng(k + n)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    w[n // 2 + 1] = w[n // 2]  # equal rows: equal scores, the lower token wins
    wt = torch.from_numpy(oracle.quantize_q4_k(w)).to(device)
    nw = torch.from_numpy((1.0 + 0.1 * rng.standard_normal(k)).astype(np.float32)).to(device)
    hs = [torch.from_numpy((rng.standard_normal(k) * (1 + i)).astype(np.float32)).to(device) for i in range(4)]
    for n_seq in (1, 2, 3, 4):
        ps = [torch.full((g,), 7.0, dtype=torch.float32, device=device) for _ in range(n_seq)]
        pt = [torch.full((g,), 7, dtype=torch.int32, device=device) for _ in range(n_seq)]
        kernels.q4k_lm_head_argmax_partial_seqs(hs[:n_seq], wt, ps, pt, norm_weight=nw)
        for i in range(n_seq):
            rs = torch.empty(g, dtype=torch.float32, device=device)
            rt = torch.empty(g, dtype=torch.int32, device=device)
            kernels.q4k_lm_head_argmax_partial(hs[i], wt, rs, rt, norm_weight=nw)
            if n_seq == 1:
                assert torch.equal(ps[i].view(torch.int32), rs.view(torch.int32)), (n_seq, i)
                assert torch.equal(pt[i], rt), (n_seq, i)
            assert _best_pair(ps[i], pt[i]) == _best_pair(rs, rt), (n_seq, i)
    # the tie: a sequence whose best row is one of the equal pair picks the lower id
    wd = oracle.dequant_q4_k(wt.cpu().numpy(), k)
    htie = torch.from_numpy((wd[n // 2] / np.linalg.norm(wd[n // 2]) * np.sqrt(k)).astype(np.float32)).to(device)
    ones = torch.ones(k, dtype=torch.float32, device=device)
    ps = [torch.empty(g, dtype=torch.float32, device=device) for _ in range(2)]
    pt = [torch.empty(g, dtype=torch.int32, device=device) for _ in range(2)]
    kernels.q4k_lm_head_argmax_partial_seqs([htie, hs[1]], wt, ps, pt, norm_weight=ones)
    eos = torch.tensor([n - 1], dtype=torch.int64, device=device)
    nxt = torch.empty(1, 1, dtype=torch.int64, device=device)
    done = torch.empty(1, dtype=torch.int32, device=device)
    kernels.token_select(ps[0], pt[0], eos, nxt, done)
    assert int(nxt.item()) == n // 2


def test_select_store_and_embedding_seqs_equal_each_sequence(device):
    """The batched select + store and the batched embedding of 4 sequences equal each sequence's own launch,
    with the sequences in different states: one stopped, one at its generated capacity, one selecting EOS."""
    from torch2vk_amd import kernels

    rng = np.random.default_rng(5)
    g, cap, n = 96, 6, 4
    eos = torch.tensor([17, 23], dtype=torch.int64, device=device)

    def state(i):
        sc = torch.from_numpy(rng.standard_normal(g).astype(np.float32)).to(device)
        tk = torch.from_numpy(rng.integers(0, 1000, g).astype(np.int32)).to(device)
        if i == 2:
            tk[int(sc.argmax())] = 23  # this sequence selects an EOS id
        gen = torch.full((cap,), -1, dtype=torch.int64, device=device)
        length = torch.tensor([cap if i == 1 else i], dtype=torch.int32, device=device)
        stopped = torch.tensor([1 if i == 3 else 0], dtype=torch.int32, device=device)
        return [sc, tk, torch.zeros(1, 1, dtype=torch.int64, device=device), torch.zeros(1, dtype=torch.int32,
                device=device), gen, length, stopped, torch.tensor([100 + i], dtype=torch.int32, device=device)]

    states = [state(i) for i in range(n)]
    mine = [[t.clone() for t in st] for st in states]
    for st in states:
        kernels.token_select_store(st[0], st[1], eos, st[2], st[3], st[4], st[5], st[6], stop_on_eos=True,
                                   advance=st[7])
    kernels.token_select_store_seqs([m[0] for m in mine], [m[1] for m in mine], eos, [m[2] for m in mine],
                                    [m[3] for m in mine], [m[4] for m in mine], [m[5] for m in mine],
                                    [m[6] for m in mine], stop_on_eos=True, advance=[m[7] for m in mine])
    for i in range(n):
        for a, b in zip(states[i], mine[i]):
            assert torch.equal(a, b), i
    assert int(states[2][3].item()) == 1 and int(states[2][6].item()) == 1  # EOS flagged and stopped
    assert int(states[1][5].item()) == cap  # at capacity: nothing appended

    dim, vocab = 1024, 300
    w = torch.from_numpy(oracle.quantize_q4_k((rng.standard_normal((vocab, dim)) * 0.05).astype(np.float32)))
    w = w.to(device)
    ids = [torch.tensor([t], dtype=torch.int64, device=device) for t in (0, 299, 17, 17)]
    outs = [torch.full((dim,), 9.0, dtype=torch.float32, device=device) for _ in ids]
    kernels.embedding_q4_k_seqs(w, ids, dim, outs)
    for t, o in zip(ids, outs):
        assert torch.equal(o, kernels.embedding_q4_k(w, t, dim)[0])

@pytest.mark.parametrize("norm", [False, True])
def test_lm_head_argmax_and_select(device, norm):
    """Fused LM-head GEMV + argmax: the index must equal the argmax of the GPU's own logits (bit-exact
    selection), and the oracle's argmax when its top-2 margin exceeds the GEMV error."""
    from torch2vk_amd import kernels

    n, k = 5000, 1024
    rng, packed, wd = _q4_problem(n, k, 99)
    h = rng.standard_normal(k).astype(np.float32)
    nw = np.ones(k, np.float32)
    x = R.bf16_round(R.rms_norm(h, nw).astype(np.float32)) if norm else R.bf16_round(h)
    wt = torch.from_numpy(packed).to(device)
    g = 64
    ps = torch.empty(g, dtype=torch.float32, device=device)
    pt = torch.empty(g, dtype=torch.int32, device=device)
    if norm:
        kernels.q4k_lm_head_argmax_partial(torch.from_numpy(h).to(device), wt, ps, pt,
                                           norm_weight=torch.from_numpy(nw).to(device))
    else:
        kernels.q4k_lm_head_argmax_partial(torch.from_numpy(x).to(device).to(torch.bfloat16), wt, ps, pt)
    eos = torch.tensor([7, 11], dtype=torch.int64, device=device)
    nxt = torch.empty(1, 1, dtype=torch.int64, device=device)
    done = torch.empty(1, dtype=torch.int32, device=device)
    kernels.token_select(ps, pt, eos, nxt, done)
    tok = int(nxt.item())
    logits = R.gemv_ref(x, wd)
    best = R.argmax_lowest(logits)
    order = np.sort(logits)[::-1]
    assert order[0] - order[1] > 1e-3, "seed gives a near tie; choose another"
    assert tok == best
    assert int(done.item()) == int(tok in (7, 11))
    # selection is exact on the GPU's own scores: recompute the scores with the plain GEMV
    if not norm:
        gl = kernels.q4k_matvec(torch.from_numpy(x).to(device).to(torch.bfloat16), wt).cpu().numpy()
        assert tok == R.argmax_lowest(gl)


def test_token_select_tie_goes_to_lowest_id(device):
    from torch2vk_amd import kernels

    scores = torch.tensor([1.0, 5.0, 5.0, 3.0, 5.0] * 300, dtype=torch.float32, device=device)
    tokens = torch.arange(scores.numel(), dtype=torch.int32, device=device).flip(0).contiguous()
    nxt = torch.empty(1, 1, dtype=torch.int64, device=device)
    done = torch.empty(1, dtype=torch.int32, device=device)
    eos = torch.tensor([2], dtype=torch.int64, device=device)
    kernels.token_select(scores, tokens, eos, nxt, done)
    ref_scores = scores.cpu().numpy()
    ref_tokens = tokens.cpu().numpy()
    best = ref_scores.max()
    expect = int(ref_tokens[ref_scores == best].min())
    assert int(nxt.item()) == expect
    assert int(done.item()) == int(expect == 2)


def test_token_store_and_advance(device):
    from torch2vk_amd import kernels

    gen = torch.full((8,), -1, dtype=torch.int64, device=device)
    length = torch.zeros(1, dtype=torch.int32, device=device)
    stopped = torch.zeros(1, dtype=torch.int32, device=device)
    pos = torch.tensor([10], dtype=torch.int32, device=device)
    nxt = torch.tensor([[42]], dtype=torch.int64, device=device)
    done = torch.zeros(1, dtype=torch.int32, device=device)
    for step in range(3):
        nxt.fill_(40 + step)
        done.fill_(1 if step == 1 else 0)
        kernels.token_store(nxt, done, gen, length, stopped, token_index_ptr=length, advance=pos)
    assert gen.cpu().tolist()[:3] == [40, 41, -1]  # stopped after the EOS at step 1
    assert int(length.item()) == 2 and int(stopped.item()) == 1 and int(pos.item()) == 13


def test_embedding_q4_k(device):
    from torch2vk_amd import kernels

    rng = np.random.default_rng(3)
    vocab, dim = 300, 1024
    w = oracle.quantize_q4_k((rng.standard_normal((vocab, dim)) * 0.02).astype(np.float32))
    ids = np.array([0, 299, 17, 17], np.int64)
    got = kernels.embedding_q4_k(torch.from_numpy(w).to(device), torch.from_numpy(ids).to(device), dim)
    np.testing.assert_array_equal(got.cpu().numpy(), oracle.dequant_q4_k(w, dim)[ids])


def _attn_case(nh, nk, s_cap, pos, seed, device, norm=True, theta=1e6):
    from torch2vk_amd import kernels

    d = 128
    rng = np.random.default_rng(seed)
    kc = R.bf16_round(rng.standard_normal((s_cap, nk, d)).astype(np.float32))
    vc = R.bf16_round(rng.standard_normal((s_cap, nk, d)).astype(np.float32))
    q = (rng.standard_normal((nh, d)) * 2).astype(np.float32)
    kn = (rng.standard_normal((nk, d)) * 2).astype(np.float32)
    vn = rng.standard_normal((nk, d)).astype(np.float32)
    qw = (1 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    kw = (1 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    # oracle: norm + rope at pos, then attention over 0..pos with the new row in the (bf16) cache
    if norm:
        cos, sin = R.rope_cos_sin(np.array([pos]), d, theta)
        qr = R.qk_norm_rope(q, qw, cos, sin)
        kr = R.qk_norm_rope(kn, kw, cos, sin)
    else:
        qr, kr = q.astype(np.float64), kn.astype(np.float64)
    kref = kc.copy()
    vref = vc.copy()
    if pos < s_cap:
        kref[pos] = R.bf16_round(kr.astype(np.float32))
        vref[pos] = R.bf16_round(vn)
    L = min(pos + 1, s_cap)
    ref = R.attention_ref(qr[None], kref[:L], vref[:L])[0]

    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)  # noqa: E731
    kct = t(kc).to(torch.bfloat16)
    vct = t(vc).to(torch.bfloat16)
    out = torch.empty(nh, d, dtype=torch.bfloat16, device=device)
    ws = kernels.attn_decode_workspace(nh, nk, d, s_cap, device)
    posb = torch.tensor([pos], dtype=torch.int32, device=device)
    kernels.attn_decode(t(q), t(kn), t(vn), kct, vct, out, posb, ws,
                        q_norm_weight=t(qw) if norm else None, k_norm_weight=t(kw) if norm else None,
                        theta=theta if norm else 0.0)
    return out.float().cpu().numpy(), ref, kct, vct, kref, vref, L


@pytest.mark.parametrize("nh,nk,s_cap,pos", [(32, 8, 4352, 4096), (16, 8, 512, 127), (32, 8, 300, 0),
                                             (32, 8, 256, 63), (32, 8, 256, 64), (16, 8, 200, 250),
                                             (8, 8, 130, 129), (64, 8, 1024, 700),
                                             # spans past one 32-row tile per wave (L > 8192 at 256 blocks)
                                             (32, 8, 9000, 8999), (32, 8, 20000, 17000), (64, 8, 9000, 8500),
                                             # one kv head: 256 blocks over it
                                             (4, 1, 3000, 2999), (8, 1, 600, 37),
                                             # GQA group 8 (4 waves a block): several 16-row tiles per wave
                                             (64, 8, 20000, 17000), (8, 1, 20000, 19999)])
def test_attn_decode(device, nh, nk, s_cap, pos):
    print(f"attn_decode nh={nh} nk={nk} S={s_cap} pos={pos}", flush=True)
    got, ref, kct, vct, kref, vref, L = _attn_case(nh, nk, s_cap, pos, seed=pos + nh, device=device)
    assert_close(got, ref, max_abs=2e-2, min_cos=0.999, what="attention out")
    # the cache holds the new row and nothing else changed
    kg = kct.float().cpu().numpy()
    vg = vct.float().cpu().numpy()
    others = np.arange(s_cap) != pos
    np.testing.assert_array_equal(kg[others], kref[others])
    np.testing.assert_array_equal(vg[others], vref[others])
    if pos < s_cap:
        # V is stored as given (one bf16 rounding); K went through norm + RoPE in fp32 (one-ulp flips allowed)
        np.testing.assert_array_equal(vg[pos], vref[pos])
        assert_close(kg[pos], kref[pos], max_abs=1e-2 * np.abs(kref[pos]).max(), min_cos=0.9999, what="new K row")


def test_attn_decode_without_norm_rope_and_reuse(device):
    """Pre-normalised inputs (the SDPA_DECODE_CACHE_WRITE_F32 contract); two calls reuse one workspace."""
    got, ref, *_ = _attn_case(32, 8, 640, 517, seed=5, device=device, norm=False)
    assert_close(got, ref, max_abs=2e-2, min_cos=0.999, what="no norm")
    got, ref, *_ = _attn_case(32, 8, 640, 100, seed=6, device=device, norm=False)
    assert_close(got, ref, max_abs=2e-2, min_cos=0.999, what="second call")


def test_attn_decode_workspace_reuse(device):
    """One workspace across calls whose chunk counts differ: stale partials of a longer call must not leak."""
    from torch2vk_amd import kernels

    nh, nk, d, s_cap = 32, 8, 128, 1100
    ws = kernels.attn_decode_workspace(nh, nk, d, s_cap, device)
    for i, pos in enumerate((1000, 5, 640, 129, 1099, 0)):
        print(f"attn_decode reuse call {i} pos={pos}", flush=True)
        rng = np.random.default_rng(100 + i)
        kc = R.bf16_round(rng.standard_normal((s_cap, nk, d)).astype(np.float32))
        vc = R.bf16_round(rng.standard_normal((s_cap, nk, d)).astype(np.float32))
        q = rng.standard_normal((nh, d)).astype(np.float32)
        kn = rng.standard_normal((nk, d)).astype(np.float32)
        vn = rng.standard_normal((nk, d)).astype(np.float32)
        kref, vref = kc.copy(), vc.copy()
        kref[pos] = R.bf16_round(kn)
        vref[pos] = R.bf16_round(vn)
        ref = R.attention_ref(q.astype(np.float64)[None], kref[:pos + 1], vref[:pos + 1])[0]
        t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)  # noqa: E731
        out = torch.empty(nh, d, dtype=torch.bfloat16, device=device)
        kernels.attn_decode(t(q), t(kn), t(vn), t(kc).to(torch.bfloat16), t(vc).to(torch.bfloat16), out,
                            torch.tensor([pos], dtype=torch.int32, device=device), ws)
        assert_close(out.float().cpu().numpy(), ref, max_abs=2e-2, min_cos=0.999, what=f"call {i}")


def test_rms_norm_and_swiglu(device):
    from torch2vk_amd import kernels

    rng = np.random.default_rng(0)
    x = (rng.standard_normal((3, 1024)) * 4).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(1024)).astype(np.float32)
    got = kernels.rms_norm(torch.from_numpy(x).to(device), torch.from_numpy(w).to(device)).cpu().numpy()
    assert_close(got, R.rms_norm(x, w), max_abs=1e-5 * math.sqrt(1024), min_cos=0.999999, what="rmsnorm")
    g = rng.standard_normal(4096).astype(np.float32)
    u = rng.standard_normal(4096).astype(np.float32)
    s = kernels.swiglu(torch.from_numpy(g).to(device), torch.from_numpy(u).to(device)).float().cpu().numpy()
    assert_close(s, R.silu_mul(g, u), max_abs=2e-2, min_cos=0.9999, what="swiglu")


@pytest.mark.parametrize("h,out_bf16", [(1024, False), (4096, True), (5120, True), (8192, False), (3000, True)])
def test_rms_norm_row_widths(device, h, out_bf16):
    """fp32 rows of 1024 .. 8192 values in whole KiB-elements take the register-resident kernel (one read of
    the row, vector loads and stores), other widths the scalar one; both against the oracle's RMSNorm."""
    from torch2vk_amd import kernels

    rng = np.random.default_rng(h)
    x = (rng.standard_normal((37, h)) * 4).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(h)).astype(np.float32)
    out = torch.empty(37, h, dtype=torch.bfloat16 if out_bf16 else torch.float32, device=device)
    got = kernels.rms_norm(torch.from_numpy(x).to(device), torch.from_numpy(w).to(device), out=out).float().cpu()
    ref = R.rms_norm(x, w)
    # fp32 rounding of the sum of squares (~1e-6 relative), then the bf16 rounding of the output (2^-9)
    tol = (2.0 ** -8 if out_bf16 else 1e-5) * float(np.abs(ref).max())
    assert_close(got.numpy(), ref, max_abs=tol, min_cos=0.99999, what=f"rmsnorm h={h}")
