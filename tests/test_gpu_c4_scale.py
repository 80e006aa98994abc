"""The prefill kernels at the full Qwen3-8B prefill configuration (8 sequences x 2048 tokens): the Q8_0 GEMM and
the gate|up + SwiGLU GEMM at M 16384, K 4096, N 12288 (a grid of 3072 tiles of 256 x 256, so the XCD-grouped
tile order runs over 64 tile rows), and causal flash attention over 8 x 2048 tokens with 32 / 8 heads of 128.
Sampled rows, columns and whole query rows are checked against fp64 references on the CPU."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from oracle import reference as R
from tests.conftest import assert_close

pytestmark = pytest.mark.gpu

M, K, N = 8 * 2048, 4096, 12288


def _sample_rows(rng):
    # first and last rows, the rows either side of tile-row and XCD-group boundaries, and random rows
    fixed = [0, 1, 255, 256, 2047, 2048, 4095, 8191, 8192, M - 257, M - 256, M - 1]
    return np.unique(np.concatenate([fixed, rng.integers(0, M, 52)]))


def _sample_cols(rng):
    fixed = [0, 1, 31, 32, 255, 256, 6143, 6144, N - 257, N - 256, N - 1]
    return np.unique(np.concatenate([fixed, rng.integers(0, N, 245)]))


@pytest.fixture(scope="module")
def c4_problem(device):
    from torch2vk_amd import kernels

    gen = torch.Generator(device=device)
    gen.manual_seed(4)
    x = torch.randn(M, K, generator=gen, device=device).to(torch.bfloat16)
    wg = kernels.quantize(torch.randn(N, K, generator=gen, device=device).mul_(0.02), "q8_0")
    wu = kernels.quantize(torch.randn(N, K, generator=gen, device=device).mul_(0.02), "q8_0")
    rng = np.random.default_rng(5)
    rows, cols = _sample_rows(rng), _sample_cols(rng)
    xr = x[torch.from_numpy(rows).to(device)].float().cpu().numpy().astype(np.float64)
    # the GEMM stages the dequantised weight tile in bf16: against x . bf16(deq W)^T only the fp32
    # accumulation order differs
    wgd = R.bf16_round(oracle.dequant_q8_0(wg.cpu().numpy(), K)).astype(np.float64)
    wud = R.bf16_round(oracle.dequant_q8_0(wu.cpu().numpy(), K)).astype(np.float64)
    return x, wg, wu, rows, cols, xr, wgd, wud


def test_gemm_q8_0_full_prefill_grid(device, c4_problem):
    from torch2vk_amd import kernels

    print(f"gemm q8_0 M={M} K={K} N={N} (3072 tiles)", flush=True)
    x, wg, _, rows, cols, xr, wgd, _ = c4_problem
    y = kernels.gemm(x, wg, "q8_0", out_dtype=torch.float32)
    torch.cuda.synchronize()
    got = y[torch.from_numpy(rows).to(device)].cpu().numpy()
    del y
    ref = xr @ wgd.T
    scale = np.abs(ref).max()
    # whole sampled rows (every column, so every tile column of those tile rows)
    assert_close(got, ref, max_abs=1e-5 * scale + 1e-6, min_cos=0.999999, what="sampled rows")
    assert np.isfinite(got).all()


def test_gemm_swiglu_q8_0_full_prefill_grid(device, c4_problem):
    from torch2vk_amd import kernels

    print(f"gemm_swiglu q8_0 M={M} K={K} F={N}", flush=True)
    x, wg, wu, rows, cols, xr, wgd, wud = c4_problem
    act = kernels.gemm_swiglu(x, wg, wu, "q8_0")
    torch.cuda.synchronize()
    got = act[torch.from_numpy(rows).to(device)].float().cpu().numpy()
    # a strided sample of every row as well: columns `cols` of all M rows
    got_cols = act[:, torch.from_numpy(cols).to(device)].float().cpu().numpy()
    del act
    g = xr @ wgd.T
    u = xr @ wud.T
    ref = g / (1.0 + np.exp(-g)) * u
    assert_close(got, ref, max_abs=8e-3 * np.abs(ref).max() + 1e-6, min_cos=0.9999, what="sampled rows")
    xall = x.float().cpu().numpy().astype(np.float64)
    gc = xall @ wgd[cols].T
    uc = xall @ wud[cols].T
    refc = gc / (1.0 + np.exp(-gc)) * uc
    assert_close(got_cols, refc, max_abs=8e-3 * np.abs(refc).max() + 1e-6, min_cos=0.9999, what="sampled columns")


def test_flash_attention_causal_8x2048(device):
    """Causal flash attention at the prefill config's shape (token-major [8, 2048, 32 | 8, 128]); whole query
    sequences of 4 (sequence, head) pairs against the fp64 reference, plus 64 sampled query rows of every head."""
    from torch2vk_amd import kernels

    b, t, nh, nk, d = 8, 2048, 32, 8, 128
    print(f"flash prefill causal b={b} t={t} nh={nh} nk={nk} d={d}", flush=True)
    gen = torch.Generator(device=device)
    gen.manual_seed(6)
    q = torch.randn(b, t, nh, d, generator=gen, device=device).to(torch.bfloat16)
    k = torch.randn(b, t, nk, d, generator=gen, device=device).to(torch.bfloat16)
    v = torch.randn(b, t, nk, d, generator=gen, device=device).to(torch.bfloat16)
    out = kernels.flash_attn_prefill(q, k, v, causal=True)
    torch.cuda.synchronize()
    qc, kc, vc, oc = (a.float().cpu().numpy() for a in (q, k, v, out))
    for bi, hi in ((0, 0), (3, 13), (5, 22), (7, 31)):
        kvh = hi * nk // nh
        ref = R.attention_ref(qc[bi, :, hi:hi + 1], kc[bi, :, kvh:kvh + 1], vc[bi, :, kvh:kvh + 1], causal_offset=0)
        assert_close(oc[bi, :, hi], ref[:, 0], max_abs=2e-2, min_cos=0.999, what=f"sequence {bi} head {hi}")
    rng = np.random.default_rng(7)
    for bi in (1, 6):
        rows = np.unique(np.concatenate([[0, 63, 64, 127, 128, t - 1], rng.integers(0, t, 58)]))
        for tq in rows:
            ref = R.attention_ref(qc[bi, tq:tq + 1], kc[bi, :tq + 1], vc[bi, :tq + 1])
            assert_close(oc[bi, tq:tq + 1], ref, max_abs=2e-2, min_cos=0.999, what=f"sequence {bi} query {tq}")


@pytest.mark.parametrize("wtype", ["q4_k", "q6_k"])
def test_gemm_k_quants_256_row_tiles(device, wtype):
    """Q4_K and Q6_K weights on the 256 x 256-tile kernel (M 4096 x N 16384: 1024 tiles, the first grid that
    takes it), whose stage loop stores the next stage at a per-format MFMA step; sampled whole rows and columns
    against x . bf16(deq W)^T in fp64."""
    from torch2vk_amd import kernels

    m, k, n = 4096, 1024, 16384
    print(f"gemm {wtype} M={m} K={k} N={n} (1024 tiles of 256 x 256)", flush=True)
    gen = torch.Generator(device=device)
    gen.manual_seed(6)
    x = torch.randn(m, k, generator=gen, device=device).to(torch.bfloat16)
    w = kernels.quantize(torch.randn(n, k, generator=gen, device=device).mul_(0.02), wtype)
    y = kernels.gemm(x, w, wtype, out_dtype=torch.float32)
    torch.cuda.synchronize()
    rng = np.random.default_rng(7)
    rows = np.unique(np.concatenate([[0, 255, 256, 2047, 2048, m - 1], rng.integers(0, m, 26)]))
    cols = np.unique(np.concatenate([[0, 255, 256, 8191, 8192, n - 1], rng.integers(0, n, 58)]))
    got_r = y[torch.from_numpy(rows).to(device)].cpu().numpy()
    got_c = y[:, torch.from_numpy(cols).to(device)].cpu().numpy()
    del y
    wd = R.bf16_round(getattr(oracle, f"dequant_{wtype}")(w.cpu().numpy(), k)).astype(np.float64)
    xall = x.float().cpu().numpy().astype(np.float64)
    ref_r = xall[rows] @ wd.T
    ref_c = xall @ wd[cols].T
    scale = max(np.abs(ref_r).max(), np.abs(ref_c).max())
    assert_close(got_r, ref_r, max_abs=1e-5 * scale + 1e-6, min_cos=0.999999, what="sampled rows")
    assert_close(got_c, ref_c, max_abs=1e-5 * scale + 1e-6, min_cos=0.999999, what="sampled columns")
