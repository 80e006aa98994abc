"""GPU parity of the MFMA flash-attention prefill kernel (through the C ABI) against the fp64 oracle.

Cases follow the reference's three prefill attention shaders: token-major causal
(LLAMA_FLASH_ATTN_F32_F16_F16), head-major causal (SDPA_CAUSAL_F32) and head-major
non-causal with an additive mask (SDPA_MASKED_F32, the Qwen3-ASR encoder).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import reference as R
from tests.conftest import assert_close

pytestmark = pytest.mark.gpu


def _qkv(rng, b, t, s, nh, nk, d):
    q = R.bf16_round(rng.standard_normal((b, t, nh, d)).astype(np.float32))
    k = R.bf16_round(rng.standard_normal((b, s, nk, d)).astype(np.float32))
    v = R.bf16_round(rng.standard_normal((b, s, nk, d)).astype(np.float32))
    return q, k, v


def _ref(q, k, v, *, causal_offset=None, mask=None):
    out = np.zeros(q.shape)
    for bi in range(q.shape[0]):
        m = None if mask is None else mask[bi if mask.shape[0] > 1 else 0]
        out[bi] = R.attention_ref(q[bi], k[bi], v[bi], causal_offset=causal_offset, mask=m)
    return out


def _dev(a, device):
    return torch.from_numpy(np.ascontiguousarray(a)).to(device).to(torch.bfloat16)


@pytest.mark.parametrize("b,t,nh,nk,d", [(2, 200, 8, 2, 128), (1, 64, 4, 4, 128), (1, 1, 32, 8, 128),
                                         (3, 130, 6, 3, 64), (1, 257, 16, 8, 128)])
def test_causal_token_major(device, b, t, nh, nk, d):
    from torch2vk_amd import kernels

    print(f"flash prefill causal token-major b={b} t={t} nh={nh} nk={nk} d={d}", flush=True)
    rng = np.random.default_rng(t + nh + d)
    q, k, v = _qkv(rng, b, t, t, nh, nk, d)
    got = kernels.flash_attn_prefill(_dev(q, device), _dev(k, device), _dev(v, device), causal=True)
    assert_close(got.float().cpu().numpy(), _ref(q, k, v, causal_offset=0), max_abs=2e-2, min_cos=0.999,
                 what="causal token-major")


def test_causal_head_major_with_offset(device):
    """Head-major tensors (transposed views) and a query block that starts after earlier keys
    (chunked prefill: queries are positions 230..299 of 300 keys)."""
    from torch2vk_amd import kernels

    print("flash prefill causal head-major offset 230", flush=True)
    rng = np.random.default_rng(7)
    b, t, s, nh, nk, d = 2, 70, 300, 8, 4, 128
    q, k, v = _qkv(rng, b, t, s, nh, nk, d)
    qh = _dev(q.transpose(0, 2, 1, 3), device).transpose(1, 2)
    kh = _dev(k.transpose(0, 2, 1, 3), device).transpose(1, 2)
    vh = _dev(v.transpose(0, 2, 1, 3), device).transpose(1, 2)
    outh = torch.empty(b, nh, t, d, dtype=torch.bfloat16, device=device)
    kernels.flash_attn_prefill(qh, kh, vh, outh.transpose(1, 2), causal=True, causal_offset=s - t)
    got = outh.transpose(1, 2).float().cpu().numpy()
    assert_close(got, _ref(q, k, v, causal_offset=s - t), max_abs=2e-2, min_cos=0.999, what="causal offset")


@pytest.mark.parametrize("d", [64, 128])
def test_masked_non_causal_head_major(device, d):
    """The ASR encoder case: non-causal, additive mask per batch (padding frames masked)."""
    from torch2vk_amd import kernels

    print(f"flash prefill masked d={d}", flush=True)
    rng = np.random.default_rng(11 + d)
    b, t, nh = 2, 150, 4
    q, k, v = _qkv(rng, b, t, t, nh, nh, d)
    mask = np.zeros((b, t, t), np.float32)
    mask[1, :, 120:] = -1e30  # batch 1: the last 30 frames are padding
    mask[0] = (rng.standard_normal((t, t)) * 0.5).astype(np.float32)  # a dense additive bias
    qh = _dev(q.transpose(0, 2, 1, 3), device).transpose(1, 2)
    kh = _dev(k.transpose(0, 2, 1, 3), device).transpose(1, 2)
    vh = _dev(v.transpose(0, 2, 1, 3), device).transpose(1, 2)
    got = kernels.flash_attn_prefill(qh, kh, vh, causal=False, mask=torch.from_numpy(mask).to(device))
    assert_close(got.float().cpu().numpy(), _ref(q, k, v, mask=mask), max_abs=2e-2, min_cos=0.999, what="masked")


def test_non_causal_cross_lengths_and_shared_mask(device):
    """t != s, one mask shared by every batch entry, explicit scale."""
    from torch2vk_amd import kernels

    print("flash prefill cross lengths", flush=True)
    rng = np.random.default_rng(3)
    b, t, s, nh, nk, d = 2, 45, 190, 8, 8, 64
    q, k, v = _qkv(rng, b, t, s, nh, nk, d)
    mask = (rng.standard_normal((1, t, s)) * 0.3).astype(np.float32)
    scale = 0.07
    got = kernels.flash_attn_prefill(_dev(q, device), _dev(k, device), _dev(v, device), causal=False,
                                     mask=torch.from_numpy(mask).to(device), scale=scale)
    # the oracle divides by sqrt(d); fold the explicit scale into q instead
    ref = _ref(q * (scale * np.sqrt(d)), k, v, mask=mask)
    assert_close(got.float().cpu().numpy(), ref, max_abs=2e-2, min_cos=0.999, what="cross lengths")


def test_fully_masked_rows_are_zero(device):
    """Negative causal offset: the first queries see no key and come out as zeros."""
    from torch2vk_amd import kernels

    rng = np.random.default_rng(5)
    q, k, v = _qkv(rng, 1, 40, 40, 2, 2, 128)
    got = kernels.flash_attn_prefill(_dev(q, device), _dev(k, device), _dev(v, device), causal=True,
                                     causal_offset=-10).float().cpu().numpy()
    assert np.all(got[0, :10] == 0.0)
    ref = _ref(q[:, 10:], k, v, causal_offset=0)
    assert_close(got[:, 10:], ref, max_abs=2e-2, min_cos=0.999, what="offset -10")


def _classes_ref(mask: np.ndarray) -> np.ndarray:
    """FA_MASK_OPT_F16's rule on 128-query x 64-key blocks: 1 all <= -FLT_MAX/2, 2 all zero, else 0."""
    b, t, s = mask.shape
    out = np.zeros((b, -(-t // 128), -(-s // 64)), np.uint8)
    lim = np.float32(1.7014117e38)
    for bi in range(b):
        for qb in range(out.shape[1]):
            for kt in range(out.shape[2]):
                blk = mask[bi, 128 * qb:128 * qb + 128, 64 * kt:64 * kt + 64]
                if blk.max() <= -lim:
                    out[bi, qb, kt] = 1
                elif blk.min() == 0 and blk.max() == 0:
                    out[bi, qb, kt] = 2
    return out


def _tile_mask(t: int, s: int, rng) -> np.ndarray:
    """Padded keys, a bidirectional block, an all-masked hole and scattered -FLT_MAX / finite entries."""
    m = np.zeros((t, s), np.float32)
    m[:, s - 70:] = -np.inf                    # padded keys: two whole tiles and a partial one
    m[128:256, 64:192] = -np.inf               # a hole of two whole tiles in the second query block
    m[:128, 192:256] = -np.finfo(np.float32).max
    m[300:, :64] = rng.standard_normal((t - 300, 64)).astype(np.float32)  # mixed
    m[5, 10] = -1.0                            # one entry makes a zero tile mixed
    return m


def test_mask_tile_classes(device):
    from torch2vk_amd import kernels

    rng = np.random.default_rng(1)
    t, s = 330, 450
    mask = np.stack([_tile_mask(t, s, rng), np.zeros((t, s), np.float32)])
    mask[1, :, 200:] = -np.inf
    tiles = kernels.fa_mask_tiles(torch.from_numpy(mask).to(device)).cpu().numpy()
    want = _classes_ref(mask)
    np.testing.assert_array_equal(tiles, want)
    assert {0, 1, 2} <= set(np.unique(want).tolist())


@pytest.mark.parametrize("shared", [False, True])
def test_mask_tiles_give_the_same_result(device, shared):
    """With the tile classes, all-masked tiles are skipped and all-zero tiles not read: bit-identical to reading
    every mask entry whenever each query sees some key (the reference's FA_MASK_OPT_F16 + flash attention)."""
    from torch2vk_amd import kernels

    rng = np.random.default_rng(2)
    b, t, s, nh, nk, d = 2, 330, 450, 8, 2, 128
    q, k, v = _qkv(rng, b, t, s, nh, nk, d)
    one = _tile_mask(t, s, rng)
    mask = one[None] if shared else np.stack([one, _tile_mask(t, s, rng)])
    mt = torch.from_numpy(mask).to(device)
    qt, kt, vt = _dev(q, device), _dev(k, device), _dev(v, device)
    with_tiles = kernels.flash_attn_prefill(qt, kt, vt, causal=False, mask=mt)
    every_entry = kernels.flash_attn_prefill(qt, kt, vt, causal=False, mask=mt, mask_tiles=False)
    assert torch.equal(with_tiles, every_entry)
    ref = _ref(q, k, v, mask=mask)
    assert_close(with_tiles.float().cpu().numpy(), ref, max_abs=2 ** -7 * max(1.0, np.abs(ref).max()),
                 min_cos=0.9999, what="tiled mask attention")
