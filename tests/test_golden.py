"""Committed golden fixtures (tests/golden/*.npz): the oracle reproduces them on the CPU, the HIP path on the GPU."""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

import oracle
from tests.conftest import assert_close

GOLDEN = Path(__file__).resolve().parent / "golden"
QUANT = [("q4_k", "q4_k_k1024.npz"), ("q6_k", "q6_k_k512.npz"), ("q8_0", "q8_0_k256.npz")]


def _load(name):
    return dict(np.load(GOLDEN / name, allow_pickle=False))


@pytest.mark.parametrize("wtype,name", QUANT)
def test_oracle_reproduces_golden_bytes(wtype, name):
    f = _load(name)
    np.testing.assert_array_equal(getattr(oracle, f"quantize_{wtype}")(f["w"]), f["packed"])
    deq = getattr(oracle, f"dequant_{wtype}")(f["packed"], f["w"].shape[1])
    np.testing.assert_allclose(np.asarray(f["x_bf16"], np.float64) @ deq.T.astype(np.float64), f["y_ref"],
                               rtol=1e-12, atol=1e-12)


@pytest.mark.gpu
@pytest.mark.parametrize("wtype,name", QUANT)
def test_gpu_quantizer_matches_golden(device, wtype, name):
    import torch

    from torch2vk_amd import kernels

    f = _load(name)
    got = kernels.quantize(torch.from_numpy(f["w"]).to(device), wtype).cpu().numpy()
    np.testing.assert_array_equal(got, f["packed"])


@pytest.mark.gpu
def test_gpu_q4k_gemv_matches_golden(device):
    import torch

    from torch2vk_amd import kernels

    f = _load("q4_k_k1024.npz")
    y = kernels.q4k_matvec(torch.from_numpy(f["x_bf16"]).to(device).to(torch.bfloat16),
                           torch.from_numpy(f["packed"]).to(device)).cpu().numpy()
    assert_close(y, f["y_ref"], max_abs=2e-4 * np.abs(f["y_ref"]).max(), min_cos=0.99999, what="golden GEMV")


@pytest.mark.gpu
def test_gpu_attention_matches_golden(device):
    import torch

    from torch2vk_amd import kernels

    f = _load("attn_decode_gqa4.npz")
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)  # noqa: E731
    kc = t(f["k_cache"]).to(torch.bfloat16)
    vc = t(f["v_cache"]).to(torch.bfloat16)
    nh, d = f["q"].shape
    s_cap, nk, _ = f["k_cache"].shape
    out = torch.empty(nh, d, dtype=torch.bfloat16, device=device)
    ws = kernels.attn_decode_workspace(nh, nk, d, s_cap, device)
    pos = torch.tensor([int(f["pos"])], dtype=torch.int32, device=device)
    kernels.attn_decode(t(f["q"]), t(f["k_new"]), t(f["v_new"]), kc, vc, out, pos, ws, q_norm_weight=t(f["q_norm"]),
                        k_norm_weight=t(f["k_norm"]), theta=float(f["theta"]))
    assert_close(out.float().cpu().numpy(), f["out_ref"], max_abs=2e-2, min_cos=0.999, what="golden attention")
