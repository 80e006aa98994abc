"""t2h_qwen3_decode_layers_noalloc (the persistent decode launch on the library's own per-GPU workspace) against
t2h_qwen3_decode_layers with a caller workspace, through the C ABI: two calls in a row, the Qwen3-8B layer shape
and then the smaller Qwen3-0.6B layer shape, each bit-identical to the workspace entry point on the same inputs."""

from __future__ import annotations

from dataclasses import replace

import pytest
import torch

pytestmark = pytest.mark.gpu


def _case(device, base, seed, pos):
    from torch2vk_amd.qwen3.model import Qwen3Decoder
    from torch2vk_amd.qwen3.weights import synthetic_weights

    cfg = replace(base, layers=2, vocab=1024, eos_token_ids=(1023,))
    w = synthetic_weights(cfg, device=device, seed=seed, std=0.02, norm_std=0.1)
    dec = Qwen3Decoder(w, max_positions=512, max_new_tokens=4, persistent=True)
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    dec.k_cache.normal_(generator=g)
    dec.v_cache.normal_(generator=g)
    h0 = torch.randn(cfg.hidden, generator=g, device=device)
    dec.position.fill_(pos)
    return cfg, dec, h0


def _call_noalloc(dec, cfg, h, status) -> int:
    from torch2vk_amd import _lib
    from torch2vk_amd._lib import stream_handle

    return _lib.lib().t2h_qwen3_decode_layers_noalloc(
        dec.layer_table.data_ptr(), int(dec.layer_table.shape[0]), cfg.hidden, cfg.mlp, cfg.heads, cfg.kv_heads,
        cfg.head_dim, dec.max_positions, h.data_ptr(), dec.position.data_ptr(), cfg.rms_eps, cfg.rope_theta,
        status.data_ptr(), stream_handle())


def test_noalloc_matches_workspace_entry(device):
    from torch2vk_amd import kernels
    from torch2vk_amd.qwen3.config import QWEN3_0_6B, QWEN3_8B

    for base, seed, pos in ((QWEN3_8B, 31, 300), (QWEN3_0_6B, 32, 57)):
        print(f"no-alloc persistent decode: {base.name} shape, 2 layers, position {pos}", flush=True)
        cfg, dec, h0 = _case(device, base, seed, pos)
        k0, v0 = dec.k_cache.clone(), dec.v_cache.clone()
        # reference: the workspace entry point
        h_ref = h0.clone()
        kernels.decode_layers(dec.layer_table, h_ref, dec.position, dec.layers_ws, dec.status, hidden=cfg.hidden,
                              mlp=cfg.mlp, nh=cfg.heads, nk=cfg.kv_heads, d=cfg.head_dim, s_cap=dec.max_positions,
                              eps=cfg.rms_eps, theta=cfg.rope_theta)
        k_ref, v_ref = dec.k_cache.clone(), dec.v_cache.clone()
        # the allocation-free entry point on the same inputs
        dec.k_cache.copy_(k0)
        dec.v_cache.copy_(v0)
        h_na = h0.clone()
        status = torch.zeros(1, dtype=torch.int32, device=device)
        torch.cuda.synchronize()
        rc = _call_noalloc(dec, cfg, h_na, status)
        torch.cuda.synchronize()
        assert rc == 0, rc
        assert int(status.item()) == 0 and int(dec.status.item()) == 0
        assert torch.equal(h_na, h_ref)
        assert torch.equal(dec.k_cache, k_ref) and torch.equal(dec.v_cache, v_ref)
        assert torch.isfinite(h_na).all()


def test_noalloc_rejects_unbuilt_shape(device):
    from torch2vk_amd import _lib

    # the Qwen3-4B layer shape (hidden 2560, MLP 9728, 32 / 8 heads) has no persistent instantiation; the null
    # table, residual and position would stop a built shape at its argument check, so nothing can launch
    status = torch.zeros(1, dtype=torch.int32, device=device)
    rc = _lib.lib().t2h_qwen3_decode_layers_noalloc(None, 2, 2560, 9728, 32, 8, 128, 512, None, None, 1e-6, 1e6,
                                                     status.data_ptr(), None)
    assert rc == 4  # T2H_ERR_UNSUPPORTED: no layout for this shape, nothing launched
