"""GPU parity of the prefill GEMMs (matrix cores, dequantised Q8_0 / Q4_K weight tiles) against the
CPU oracle, through the C ABI."""

from __future__ import annotations

from contextlib import contextmanager

import numpy as np
import pytest
import torch

import oracle
from oracle import reference as R
from tests.conftest import assert_close

pytestmark = pytest.mark.gpu


@contextmanager
def _in_loop():
    """The quantized GEMM dequantising inside its tile loop at any M: without this, from
    kernels.DEQUANT_FIRST_ROWS rows it dequantises once and runs the bf16-row kernels it is compared with."""
    from torch2vk_amd import kernels

    saved = kernels.DEQUANT_FIRST_ROWS
    kernels.DEQUANT_FIRST_ROWS = 0
    try:
        yield
    finally:
        kernels.DEQUANT_FIRST_ROWS = saved


def _problem(wtype, m, k, n, seed):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    w[0] = 0.0
    if n > 3:
        w[3] = np.abs(w[3]) * 40
    packed = getattr(oracle, f"quantize_{wtype}")(w)
    wd = getattr(oracle, f"dequant_{wtype}")(packed, k)
    x = R.bf16_round(rng.standard_normal((m, k)).astype(np.float32))
    return rng, packed, wd, x


# (m, k, n): exact tiles, ragged M and N (partial 256-tiles), a handful of tokens, long K
CASES = [("q8_0", 256, 256, 256), ("q8_0", 300, 1024, 520), ("q8_0", 17, 2048, 1024), ("q8_0", 512, 4096, 768),
         ("q4_k", 256, 256, 256), ("q4_k", 300, 1024, 520), ("q4_k", 9, 4096, 1024), ("q4_k", 640, 3072, 256),
         ("q6_k", 256, 256, 256), ("q6_k", 300, 1024, 520), ("q6_k", 17, 4096, 1024), ("q6_k", 700, 3072, 384)]


@pytest.mark.parametrize("splits", [1, None], ids=["one_pass", "auto_split"])
@pytest.mark.parametrize("wtype,m,k,n", CASES)
def test_gemm_matches_oracle(device, wtype, m, k, n, splits):
    """splits 1: the one-pass kernel; None: the wrapper's choice (small grids split K: t2h_gemm_splitk)."""
    from torch2vk_amd import kernels

    print(f"gemm {wtype} M={m} K={k} N={n} splits={kernels.gemm_splits(m, n, k) if splits is None else 1}",
          flush=True)
    rng, packed, wd, x = _problem(wtype, m, k, n, m + k + n)
    xt = torch.from_numpy(x).to(device).to(torch.bfloat16)
    wt = torch.from_numpy(packed).to(device)
    got = kernels.gemm(xt, wt, wtype, out_dtype=torch.float32, splits=splits).cpu().numpy()
    # the weight tile is dequantised to bf16: against x . bf16(deq W)^T only fp32 accumulation differs,
    # which pins the tile layout and the dequantisation exactly
    ref_tile = x.astype(np.float64) @ R.bf16_round(wd.astype(np.float32)).astype(np.float64).T
    scale = np.abs(ref_tile).max()
    assert_close(got, ref_tile, max_abs=1e-5 * scale + 1e-6, min_cos=0.999999, what="vs bf16 tile")
    # and against the exact dequantised weights: the stated prefill tolerance
    ref = x.astype(np.float64) @ wd.astype(np.float64).T
    assert_close(got, ref, max_abs=1e-2 * np.abs(ref).max(), min_cos=0.9999, what="vs fp64 oracle")
    # bf16 output and the residual epilogue (in place)
    got16 = kernels.gemm(xt, wt, wtype, splits=splits).float().cpu().numpy()
    assert_close(got16, ref_tile, max_abs=1e-2 * scale, min_cos=0.9999, what="bf16 out")
    res = rng.standard_normal((m, n)).astype(np.float32)
    rt = torch.from_numpy(res).to(device)
    kernels.gemm(xt, wt, wtype, out=rt, residual=rt, splits=splits)
    assert_close(rt.cpu().numpy(), ref_tile + res, max_abs=1e-5 * scale + 1e-5, min_cos=0.999999, what="residual")


def test_gemm_rejects_bad_shapes(device):
    from torch2vk_amd import _lib, kernels

    x = torch.zeros(4, 1056, dtype=torch.bfloat16, device=device)
    w = torch.zeros(64, 1056 // 32 * 34, dtype=torch.uint8, device=device)
    with pytest.raises(ValueError, match="K % 64"):
        kernels.gemm(x, w, "q8_0")
    y = torch.empty(4, 64, dtype=torch.float32, device=device)
    st = _lib.lib().t2h_q8_0_gemm(x.data_ptr(), w.data_ptr(), y.data_ptr(), 0, None, 4, 1056, 64, None)
    assert st == 2


@pytest.mark.parametrize("splits", [1, None], ids=["one_pass", "auto_split"])
@pytest.mark.parametrize("wtype,m,k,n", [("q8_0", 300, 1024, 520), ("q4_k", 17, 2048, 1024), ("q8_0", 700, 512, 96),
                                         ("q6_k", 260, 1024, 384), ("q4_k", 1030, 4096, 768)])
def test_gemm_swiglu_matches_oracle(device, wtype, m, k, n, splits):
    """Gate and up products with SwiGLU in the epilogue, against silu(x Wg^T) * (x Wu^T) on the bf16 tiles."""
    from torch2vk_amd import kernels

    print(f"gemm_swiglu {wtype} M={m} K={k} F={n}", flush=True)
    rng, pg, wg, x = _problem(wtype, m, k, n, m + k)
    wu = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    pu = getattr(oracle, f"quantize_{wtype}")(wu)
    wud = getattr(oracle, f"dequant_{wtype}")(pu, k)
    xd = x.astype(np.float64)
    g = xd @ R.bf16_round(wg.astype(np.float32)).astype(np.float64).T
    u = xd @ R.bf16_round(wud.astype(np.float32)).astype(np.float64).T
    ref = g / (1.0 + np.exp(-g)) * u
    xt = torch.from_numpy(x).to(device).to(torch.bfloat16)
    got = kernels.gemm_swiglu(xt, torch.from_numpy(pg).to(device), torch.from_numpy(pu).to(device), wtype,
                              splits=splits)
    assert_close(got.float().cpu().numpy(), ref, max_abs=8e-3 * np.abs(ref).max() + 1e-6, min_cos=0.9999,
                 what="gemm_swiglu")


@pytest.mark.parametrize("wtype,m,k,n,splits", [("q8_0", 128, 2048, 1024, 16), ("q4_k", 100, 3072, 1024, 5),
                                                ("q6_k", 37, 1024, 4096, 3), ("q8_0", 512, 1024, 4096, 4),
                                                ("q4_k", 483, 3072, 1024, 16)])
def test_gemm_splitk_equals_one_pass(device, wtype, m, k, n, splits):
    """Split-K (parts of uneven stage counts included) against the one-pass kernel on the same inputs: the same
    products summed in another fp32 order, so within fp32 rounding of the sum; the residual epilogue in place,
    the bf16 output, and the SwiGLU form (gate | up products reduced, then silu(g) u)."""
    from torch2vk_amd import kernels

    print(f"split-K {wtype} M={m} K={k} N={n} splits={splits}", flush=True)
    g = torch.Generator(device=device)
    g.manual_seed(m + n + splits)
    x = torch.randn(m, k, generator=g, device=device).to(torch.bfloat16)
    w = kernels.quantize(torch.randn(n, k, generator=g, device=device) * 0.02, wtype)
    one = kernels.gemm(x, w, wtype, out_dtype=torch.float32, splits=1)
    got = kernels.gemm(x, w, wtype, out_dtype=torch.float32, splits=splits)
    scale = one.abs().max().item()
    assert (got - one).abs().max().item() <= 1e-5 * scale
    res = torch.randn(m, n, generator=g, device=device)
    r1, r2 = res.clone(), res.clone()
    kernels.gemm(x, w, wtype, out=r1, residual=r1, splits=1)
    kernels.gemm(x, w, wtype, out=r2, residual=r2, splits=splits)
    assert (r1 - r2).abs().max().item() <= 1e-5 * (scale + res.abs().max().item())
    b1 = kernels.gemm(x, w, wtype, splits=1).float()
    b2 = kernels.gemm(x, w, wtype, splits=splits).float()
    # bf16 roundings of fp32 values within 1e-5 of the scale: one bf16 step apart, or that absolute error
    assert ((b1 - b2).abs() <= 2 ** -7 * b1.abs() + 2e-5 * scale).all()
    wu = kernels.quantize(torch.randn(n, k, generator=g, device=device) * 0.02, wtype)
    s1 = kernels.gemm_swiglu(x, w, wu, wtype, splits=1).float()
    s2 = kernels.gemm_swiglu(x, w, wu, wtype, splits=splits).float()
    assert ((s1 - s2).abs() <= 2 ** -7 * s1.abs() + 1e-4 * s1.abs().max()).all()
    torch.cuda.synchronize()


def test_gemm_splitk_rejects_bad_arguments(device):
    from torch2vk_amd import _lib

    lib = _lib.lib()
    x = torch.zeros(4, 256, dtype=torch.bfloat16, device=device)
    w = torch.zeros(64, 256 // 32 * 34, dtype=torch.uint8, device=device)
    y = torch.empty(4, 64, dtype=torch.float32, device=device)
    need = int(lib.t2h_gemm_splitk_bytes(4, 64, 2, 0))
    assert need == 2 * 4 * 64 * 4
    assert int(lib.t2h_gemm_splitk_bytes(4, 100, 2, 1)) == 2 * 4 * 256 * 4  # gate | up rows in whole tiles
    part = torch.empty(need // 4, dtype=torch.float32, device=device)
    args = lambda splits, nbytes: (8, x.data_ptr(), w.data_ptr(), None, None, 0, y.data_ptr(), 0, None, 4, 256, 64,
                                   256, splits, part.data_ptr(), nbytes, None)
    assert lib.t2h_gemm_splitk(*args(2, need - 4)) == 6     # workspace too small
    assert lib.t2h_gemm_splitk(*args(5, need * 4)) == 5     # more parts than 64-wide stages (4)
    assert lib.t2h_gemm_splitk(*args(0, need)) == 5
    assert lib.t2h_gemm_splitk(*args(2, need)) == 0
    torch.cuda.synchronize()


@pytest.mark.parametrize("wtype,m,k,n", [("q8_0", 300, 1024, 520), ("q8_0", 1024, 4096, 768), ("q4_k", 300, 1024, 520),
                                         ("q4_k", 17, 2048, 1024), ("q6_k", 700, 3072, 384)])
def test_dequantize_bf16_gemm_equals_quantized_gemm(device, wtype, m, k, n):
    """Weights dequantised once (t2h_dequantize_bf16) hold the very bf16 values the quantized GEMM builds in its
    LDS tiles: the bf16-weight GEMM (t2h_bf16_gemm, and the SwiGLU form) over them is bit-identical to the
    quantized GEMM, one pass and split-K; and the dequantised rows are the oracle's dequantisation rounded to
    bf16 (bit-equal for Q8_0, whose fp32 values d * q are exact; within one bf16 step for the K types, whose
    fp32 products may round before the bf16 rounding in a different order)."""
    from torch2vk_amd import kernels

    rng, packed, wd, x = _problem(wtype, m, k, n, 31)
    w = torch.from_numpy(packed).to(device)
    wb = kernels.dequantize_bf16(w, wtype, k)
    ref_b = torch.from_numpy(wd).to(torch.bfloat16)
    if wtype == "q8_0":
        assert torch.equal(wb.cpu().view(torch.int16), ref_b.view(torch.int16))
    else:
        diff = (wb.cpu().float() - ref_b.float()).abs()
        assert (diff <= 2 ** -7 * ref_b.float().abs()).all()
    xt = torch.from_numpy(x).to(device).to(torch.bfloat16)
    for splits in (1, None):
        yq = kernels.gemm(xt, w, wtype, out_dtype=torch.float32, splits=splits)
        yb = kernels.gemm(xt, wb, "bf16", out_dtype=torch.float32, splits=splits)
        torch.testing.assert_close(yb, yq, rtol=0, atol=0)
    n_ff = n // 2
    g, u = w[:n_ff].contiguous(), w[n_ff:2 * n_ff].contiguous()
    gb, ub = wb[:n_ff].contiguous(), wb[n_ff:2 * n_ff].contiguous()
    for splits in (1, None):
        aq = kernels.gemm_swiglu(xt, g, u, wtype, splits=splits)
        ab = kernels.gemm_swiglu(xt, gb, ub, "bf16", splits=splits)
        torch.testing.assert_close(ab, aq, rtol=0, atol=0)


def test_bf16_gemm_matches_fp32_reference(device):
    """bf16 weights straight from a model (no quantization), ragged M, N and the K tail of a 64-wide stage
    boundary: against the fp32 product of the same bf16 operands."""
    from torch2vk_amd import kernels

    g = torch.Generator(device=device)
    g.manual_seed(5)
    m, k, n = 333, 1088, 700
    x = torch.randn(m, k, generator=g, device=device).to(torch.bfloat16)
    w = (torch.randn(n, k, generator=g, device=device) * 0.05).to(torch.bfloat16)
    y = kernels.gemm(x, w, "bf16", out_dtype=torch.float32, splits=1)
    ref = x.float() @ w.float().t()
    err = (y - ref).abs().max().item()
    assert err <= 1e-4 * ref.abs().max().item(), err


@pytest.mark.parametrize("wtype,m,k,n", [("q8_0", 4000, 256, 16384), ("q4_k", 4096, 512, 16200)])
def test_bf16_gemm_large_grid_equals_quantized_gemm(device, wtype, m, k, n):
    """The prefill's grid size (>= 1024 tiles of 256 x 256, the 256-row tile loop), ragged M (4000) and N
    (16200): bf16 weights dequantised once give the quantized GEMM's bits in the plain, bf16, residual and SwiGLU
    epilogues."""
    from torch2vk_amd import kernels

    g = torch.Generator(device=device)
    g.manual_seed(9)
    w = kernels.quantize(torch.randn(n, k, generator=g, device=device) * 0.02, wtype)
    wb = kernels.dequantize_bf16(w, wtype, k)
    x = torch.randn(m, k, generator=g, device=device).to(torch.bfloat16)
    with _in_loop():
        yq = kernels.gemm(x, w, wtype, out_dtype=torch.float32, splits=1)
    yb = kernels.gemm(x, wb, "bf16", out_dtype=torch.float32, splits=1)
    torch.testing.assert_close(yb, yq, rtol=0, atol=0)
    with _in_loop():
        yq16 = kernels.gemm(x, w, wtype, out_dtype=torch.bfloat16, splits=1)
    yb16 = kernels.gemm(x, wb, "bf16", out_dtype=torch.bfloat16, splits=1)
    torch.testing.assert_close(yb16, yq16, rtol=0, atol=0)
    r = torch.randn(m, n, generator=g, device=device)
    rq, rb = r.clone(), r.clone()
    with _in_loop():
        kernels.gemm(x, w, wtype, out=rq, residual=rq, splits=1)
    kernels.gemm(x, wb, "bf16", out=rb, residual=rb, splits=1)
    torch.testing.assert_close(rb, rq, rtol=0, atol=0)
    del yq, yb, yq16, yb16, r, rq, rb
    n_ff = n // 2
    with _in_loop():
        aq = kernels.gemm_swiglu(x, w[:n_ff].contiguous(), w[n_ff:2 * n_ff].contiguous(), wtype, splits=1)
    ab = kernels.gemm_swiglu(x, wb[:n_ff].contiguous(), wb[n_ff:2 * n_ff].contiguous(), "bf16", splits=1)
    torch.testing.assert_close(ab, aq, rtol=0, atol=0)


@pytest.mark.parametrize("m,n", [(4096, 8192), (16384, 1024), (4000, 9000)])
def test_bf16_ring_grid_sizes_equal_quantized_gemm(device, m, n):
    """The ring kernel's smaller grids: 512 tiles of 256 x 256, exactly 256 (one round), and ragged M and N at
    576 tiles: the quantized GEMM's bits, fp32, bf16, residual and SwiGLU."""
    from torch2vk_amd import kernels

    g = torch.Generator(device=device)
    g.manual_seed(m + n)
    k = 320
    w = kernels.quantize(torch.randn(n, k, generator=g, device=device) * 0.05, "q8_0")
    wb = kernels.dequantize_bf16(w, "q8_0", k)
    x = torch.randn(m, k, generator=g, device=device).to(torch.bfloat16)
    for dt in (torch.float32, torch.bfloat16):
        with _in_loop():
            yq = kernels.gemm(x, w, "q8_0", out_dtype=dt, splits=1)
        yb = kernels.gemm(x, wb, "bf16", out_dtype=dt, splits=1)
        torch.testing.assert_close(yb, yq, rtol=0, atol=0)
    r = torch.randn(m, n, generator=g, device=device)
    rq, rb = r.clone(), r.clone()
    with _in_loop():
        kernels.gemm(x, w, "q8_0", out=rq, residual=rq, splits=1)
    kernels.gemm(x, wb, "bf16", out=rb, residual=rb, splits=1)
    torch.testing.assert_close(rb, rq, rtol=0, atol=0)
    n_ff = n // 2
    with _in_loop():
        aq = kernels.gemm_swiglu(x, w[:n_ff].contiguous(), w[n_ff:2 * n_ff].contiguous(), "q8_0", splits=1)
    ab = kernels.gemm_swiglu(x, wb[:n_ff].contiguous(), wb[n_ff:2 * n_ff].contiguous(), "bf16", splits=1)
    torch.testing.assert_close(ab, aq, rtol=0, atol=0)


@pytest.mark.parametrize("k", [64, 128, 192, 1088])
def test_bf16_large_grid_stage_counts_equal_quantized_gemm(device, k):
    """The large-grid bf16 kernel (two LDS stages of 64 K, the last stage peeled, the stage after the end loaded
    into a buffer nothing reads) at 1, 2, 3 and 17 stages: the quantized GEMM's bits, plain and SwiGLU."""
    from torch2vk_amd import kernels

    g = torch.Generator(device=device)
    g.manual_seed(k)
    m, n = 4096, 16384
    w = kernels.quantize(torch.randn(n, k, generator=g, device=device) * 0.05, "q8_0")
    wb = kernels.dequantize_bf16(w, "q8_0", k)
    x = torch.randn(m, k, generator=g, device=device).to(torch.bfloat16)
    with _in_loop():
        yq = kernels.gemm(x, w, "q8_0", out_dtype=torch.float32, splits=1)
    yb = kernels.gemm(x, wb, "bf16", out_dtype=torch.float32, splits=1)
    torch.testing.assert_close(yb, yq, rtol=0, atol=0)
    del yq, yb
    n_ff = n // 2
    with _in_loop():
        aq = kernels.gemm_swiglu(x, w[:n_ff].contiguous(), w[n_ff:].contiguous(), "q8_0", splits=1)
    ab = kernels.gemm_swiglu(x, wb[:n_ff].contiguous(), wb[n_ff:].contiguous(), "bf16", splits=1)
    torch.testing.assert_close(ab, aq, rtol=0, atol=0)


def test_q8_0_linear_dequantise_once_equals_in_loop(device):
    """The encoder's linears at M >= 4096 (bias + GELU, and fp32 residual) over Q8_0 weights dequantised once
    (t2h_bf16_linear) give the in-loop GEMM's bits; weights shorter than x's rows (w_k < K) keep the in-loop
    path."""
    from torch2vk_amd import kernels

    g = torch.Generator(device=device)
    g.manual_seed(13)
    m, k, n = 4500, 1024, 1536
    x = torch.randn(m, k, generator=g, device=device).to(torch.bfloat16)
    w = kernels.quantize(torch.randn(n, k, generator=g, device=device) * 0.03, "q8_0")
    bias = torch.randn(n, generator=g, device=device)
    saved = kernels.DEQUANT_FIRST_ROWS
    try:
        kernels.DEQUANT_FIRST_ROWS = 0
        ref = kernels.q8_0_linear(x, w, bias=bias, act="gelu")
        r0 = torch.randn(m, n, generator=g, device=device)
        ref_res = kernels.q8_0_linear(x, w, bias=bias, out=r0.clone(), out_dtype=torch.float32, residual=None)
        ref_res2 = r0.clone()
        kernels.q8_0_linear(x, w, out=ref_res2, out_dtype=torch.float32, residual=ref_res2)
        kernels.DEQUANT_FIRST_ROWS = 4096
        got = kernels.q8_0_linear(x, w, bias=bias, act="gelu")
        got_res = kernels.q8_0_linear(x, w, bias=bias, out=r0.clone(), out_dtype=torch.float32, residual=None)
        got_res2 = r0.clone()
        kernels.q8_0_linear(x, w, out=got_res2, out_dtype=torch.float32, residual=got_res2)
    finally:
        kernels.DEQUANT_FIRST_ROWS = saved
    torch.testing.assert_close(got, ref, rtol=0, atol=0)
    torch.testing.assert_close(got_res, ref_res, rtol=0, atol=0)
    torch.testing.assert_close(got_res2, ref_res2, rtol=0, atol=0)
