"""BASELINE configs[2] at full depth: the 36-layer Qwen3-8B shape (vocab 151936, uniform Q4_K) decoding with the
persistent layers kernel from a bf16 KV cache prefilled to 4096 positions with N(0,1) keys and values, as the
headline bench runs it; every greedy token against the CPU oracle decoder started from the same cache, checked
step by step over the GPU's own KV history.  The oracle holds the dequantized weights in fp32 (~33 GB of host
memory) and reads them all once per step."""

from __future__ import annotations

import time

import numpy as np
import pytest
import torch

from oracle.qwen3_check import check_greedy_tokens, decoder_step_logits, dense_weights
from oracle.reference import Qwen3Shape

pytestmark = [pytest.mark.gpu, pytest.mark.timeout(900)]


def test_c3_full_depth_decode_from_kv4096_matches_oracle(device):
    from torch2vk_amd.qwen3.config import QWEN3_8B
    from torch2vk_amd.qwen3.model import Qwen3Decoder
    from torch2vk_amd.qwen3.weights import matrix_shapes, synthetic_weights

    cfg = QWEN3_8B
    t0 = time.time()
    print("C3 full depth: quantizing the 36-layer 8B-shape weights on the GPU", flush=True)
    w = synthetic_weights(cfg, device=device, seed=3, std=0.02, norm_std=0.1)
    start = 4096
    dec = Qwen3Decoder(w, max_positions=start + 32, max_new_tokens=16)
    assert dec.persistent
    dec.stop_on_eos = False
    g = torch.Generator(device=device)
    g.manual_seed(44)
    dec.k_cache[:, :start].normal_(generator=g)
    dec.v_cache[:, :start].normal_(generator=g)
    prompt = [1517, 98304]
    dec.prefill(torch.tensor(prompt), start=start)
    dec.run_steps(7, steps_per_graph=4, use_graph=True)
    toks = dec.generated[:int(dec.length.item())].tolist()
    dec.check_status()
    assert int(dec.status.item()) == 0 and len(toks) == 8
    print(f"GPU tokens {toks} ({time.time() - t0:.1f} s); dequantizing the oracle's weights", flush=True)
    shape = Qwen3Shape(hidden=cfg.hidden, layers=cfg.layers, heads=cfg.heads, kv_heads=cfg.kv_heads,
                       head_dim=cfg.head_dim, mlp=cfg.mlp, vocab=cfg.vocab, rope_theta=cfg.rope_theta)
    dense = dense_weights({k: v.cpu().numpy() for k, v in w.packed.items()}, w.types,
                          {k: v.cpu().numpy() for k, v in w.norms.items()}, matrix_shapes(cfg))
    print(f"oracle weights ready ({time.time() - t0:.1f} s); replaying", flush=True)
    kv = (dec.k_cache[:, :start].cpu(), dec.v_cache[:, :start].cpu())
    stats = check_greedy_tokens(shape, dense, prompt, toks, start=start, kv_init=kv,
                                kv_history=(dec.k_cache, dec.v_cache), gpu_logits=decoder_step_logits(dec),
                                label="C3 36 layers from KV 4096")
    print(f"{stats} ({time.time() - t0:.1f} s)", flush=True)
    assert stats["steps"] == 8
    assert np.isfinite(stats["min_margin"])
