"""GPU parity of the Q6_K and Q8_0 decode GEMVs and the Q6_K LM head against the CPU oracle
(every call goes through the C ABI)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from oracle import reference as R
from tests.conftest import assert_close

pytestmark = pytest.mark.gpu


def _problem(wtype, n, k, seed, special=True):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    if special and n >= 8:
        w[0] = 0.0                                         # d = 0
        w[1] = 0.37                                        # constant row
        w[2] = np.abs(w[2]) * 50                           # all positive, large
        w[3] = np.where(np.arange(k) % 32 == 5, -7.0, 0.0)  # one spike per 32
    packed = getattr(oracle, f"quantize_{wtype}")(w)
    wd = getattr(oracle, f"dequant_{wtype}")(packed, k)
    return rng, packed, wd


# (n, k): row-groups of 4 and 2 rows (short rows), partly idle lanes (K=3072: 48 pieces),
# the 8B shapes (K=4096, 12288) and two and three steps per row
Q6_CASES = [(64, 1024), (96, 2048), (48, 3072), (256, 4096), (40, 8192), (64, 12288)]
Q8_CASES = [(20, 512), (64, 1024), (33, 1056), (96, 3072), (128, 4096), (32, 12288)]


@pytest.mark.parametrize("wtype,n,k", [("q6_k", n, k) for n, k in Q6_CASES] + [("q8_0", n, k) for n, k in Q8_CASES])
def test_qx_matvec(device, wtype, n, k):
    from torch2vk_amd import kernels

    print(f"{wtype} matvec N={n} K={k}", flush=True)
    rng, packed, wd = _problem(wtype, n, k, n * 7 + k)
    x = R.bf16_round(rng.standard_normal(k).astype(np.float32))
    ref = R.gemv_ref(x, wd)
    wt = torch.from_numpy(packed).to(device)
    xt = torch.from_numpy(x).to(device).to(torch.bfloat16)
    scale = np.abs(ref).max()
    got = kernels.qx_matvec(xt, wt, wtype).cpu().numpy()
    assert_close(got, ref, max_abs=2e-4 * scale + 1e-6, min_cos=0.99999, what=f"{wtype} f32 out")
    res = rng.standard_normal(n).astype(np.float32)
    rt = torch.from_numpy(res).to(device)
    kernels.qx_matvec(xt, wt, wtype, out=rt, residual=rt)
    assert_close(rt.cpu().numpy(), ref + res, max_abs=2e-4 * scale + 1e-5, min_cos=0.99999, what="residual")
    got16 = kernels.qx_matvec(xt, wt, wtype, out_dtype=torch.bfloat16).float().cpu().numpy()
    assert_close(got16, ref, max_abs=1e-2 * scale + 1e-6, min_cos=0.9999, what="bf16 out")


@pytest.mark.parametrize("wtype", ["q6_k", "q8_0"])
def test_qx_matvec_multi_token(device, wtype):
    from torch2vk_amd import kernels

    n, k, m = 128, 2048, 3
    rng, packed, wd = _problem(wtype, n, k, 11)
    x = R.bf16_round(rng.standard_normal((m, k)).astype(np.float32))
    ref = R.gemv_ref(x, wd)
    got = kernels.qx_matvec(torch.from_numpy(x).to(device).to(torch.bfloat16), torch.from_numpy(packed).to(device),
                            wtype).cpu().numpy()
    assert_close(got, ref, max_abs=2e-4 * np.abs(ref).max(), min_cos=0.99999, what=f"{wtype} M=3")


def test_q8_0_matches_fp16_activation_semantics(device):
    """Q8_0 runs on fp16 activations, like the reference: a bf16 x whose values are not fp16-exact
    (below fp16's normal range) is rounded to fp16 first."""
    from torch2vk_amd import kernels

    n, k = 64, 1024
    rng, packed, wd = _problem("q8_0", n, k, 5, special=False)
    x = R.bf16_round((rng.standard_normal(k) * np.where(np.arange(k) % 3 == 0, 1e-6, 1.0)).astype(np.float32))
    x16 = x.astype(np.float16).astype(np.float32)
    ref = R.gemv_ref(x16, wd)
    got = kernels.qx_matvec(torch.from_numpy(x).to(device).to(torch.bfloat16), torch.from_numpy(packed).to(device),
                            "q8_0").cpu().numpy()
    assert_close(got, ref, max_abs=2e-4 * np.abs(ref).max(), min_cos=0.99999, what="fp16 x")


@pytest.mark.parametrize("k,n", [(1024, 1024), (4096, 1024), (12288, 64)])
def test_q6k_rmsnorm_prologue(device, k, n):
    from torch2vk_amd import kernels

    rng, packed, wd = _problem("q6_k", n, k, k + 3)
    h = (rng.standard_normal(k) * 3).astype(np.float32)
    nw = (1 + 0.1 * rng.standard_normal(k)).astype(np.float32)
    xn = R.bf16_round(R.rms_norm(h, nw).astype(np.float32))
    ref = R.gemv_ref(xn, wd)
    got = kernels.qx_matvec(torch.from_numpy(h).to(device), torch.from_numpy(packed).to(device), "q6_k",
                            norm_weight=torch.from_numpy(nw).to(device)).cpu().numpy()
    assert_close(got, ref, max_abs=2e-3 * np.abs(ref).max(), min_cos=0.9999, what="q6_k rmsnorm")


@pytest.mark.parametrize("norm", [False, True])
def test_q6k_lm_head_argmax(device, norm):
    """Q6_K LM head + argmax: equals the oracle's argmax (top-2 margin above the GEMV error) and the
    argmax of the GPU's own Q6_K logits."""
    from torch2vk_amd import kernels

    n, k = 5000, 1024
    rng, packed, wd = _problem("q6_k", n, k, 123, special=False)
    h = rng.standard_normal(k).astype(np.float32)
    nw = np.ones(k, np.float32)
    x = R.bf16_round(R.rms_norm(h, nw).astype(np.float32)) if norm else R.bf16_round(h)
    wt = torch.from_numpy(packed).to(device)
    g = 40
    ps = torch.empty(g, dtype=torch.float32, device=device)
    pt = torch.empty(g, dtype=torch.int32, device=device)
    if norm:
        kernels.lm_head_argmax_partial(torch.from_numpy(h).to(device), wt, "q6_k", ps, pt,
                                       norm_weight=torch.from_numpy(nw).to(device))
    else:
        kernels.lm_head_argmax_partial(torch.from_numpy(x).to(device).to(torch.bfloat16), wt, "q6_k", ps, pt)
    eos = torch.tensor([3], dtype=torch.int64, device=device)
    nxt = torch.empty(1, 1, dtype=torch.int64, device=device)
    done = torch.empty(1, dtype=torch.int32, device=device)
    kernels.token_select(ps, pt, eos, nxt, done)
    tok = int(nxt.item())
    logits = R.gemv_ref(x, wd)
    order = np.sort(logits)[::-1]
    assert order[0] - order[1] > 1e-3, "seed gives a near tie; choose another"
    assert tok == R.argmax_lowest(logits)
    if not norm:
        gl = kernels.qx_matvec(torch.from_numpy(x).to(device).to(torch.bfloat16), wt, "q6_k").cpu().numpy()
        assert tok == R.argmax_lowest(gl)


def test_q6k_lm_head_tie_goes_to_lowest_row(device):
    """Duplicated rows give exactly equal scores; the lowest row id must win across blocks."""
    from torch2vk_amd import kernels

    n, k = 4096, 1024
    rng, packed, _ = _problem("q6_k", n, k, 77, special=False)
    x = R.bf16_round(rng.standard_normal(k).astype(np.float32))
    wd = oracle.dequant_q6_k(packed, k)
    best = int(R.argmax_lowest(R.gemv_ref(x, wd)))
    for r in (best + 1 + 1000) % n, (best + 3000) % n, n - 1:
        packed[r] = packed[best]
    xt = torch.from_numpy(x).to(device).to(torch.bfloat16)
    wt = torch.from_numpy(packed).to(device)
    ps = torch.empty(64, dtype=torch.float32, device=device)
    pt = torch.empty(64, dtype=torch.int32, device=device)
    kernels.lm_head_argmax_partial(xt, wt, "q6_k", ps, pt)
    nxt = torch.empty(1, 1, dtype=torch.int64, device=device)
    done = torch.empty(1, dtype=torch.int32, device=device)
    kernels.token_select(ps, pt, torch.tensor([0], dtype=torch.int64, device=device), nxt, done)
    copies = sorted({best, (best + 1 + 1000) % n, (best + 3000) % n, n - 1})
    assert int(nxt.item()) == copies[0]
