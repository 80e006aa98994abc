"""BASELINE configs[4] at the depth and size it is benchmarked at (bench.py --config asr), against the CPU oracle.

* The encoder: 24 layers, hidden 1024, 16 heads of 64, FFN 4096, Q8_0 linears, over 4 utterances x 1500 frames
  of N(0,1) features with attention within each utterance (t2h_flash_attn_segments), then ln_post / proj1 /
  proj2.  Utterances are independent, so the oracle runs two of them (the first and the last) alone.
* The decoder: the 28-layer Qwen3-0.6B shape (vocab 151936, uniform Q4_K) as a Qwen3DecoderGroup of 4
  sequences, each prompt 1507 positions with one utterance's encoder states injected at the audio placeholder
  positions, prefilled as one batch, then 16 greedy tokens of the 4 sequences in one persistent launch per step
  (t2h_qwen3_decode_layers_seqs).  Every sequence's status word stays clear and its tokens are checked against
  the oracle decoder given the same injected embeddings.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import asr as oasr
from oracle.qwen3_check import check_greedy_tokens, decoder_step_logits, dense_weights
from oracle.reference import Qwen3Shape
from tests.conftest import assert_close

pytestmark = [pytest.mark.gpu, pytest.mark.timeout(900)]

NB, FRAMES, NEW_TOKENS = 4, 1500, 16


@pytest.fixture(scope="module")
def c5_encoder(device):
    """The GPU encoder's output for the benchmark's input, with the weights and input it came from."""
    from torch2vk_amd.qwen3_asr.config import ASR_C5_ENCODER
    from torch2vk_amd.qwen3_asr.encoder import Qwen3AudioEncoder, quantize_audio_weights, synthetic_audio_dense

    cfg = ASR_C5_ENCODER
    print(f"c5 encoder: {cfg.layers} x {cfg.d_model}, {NB} x {FRAMES} frames", flush=True)
    enc = Qwen3AudioEncoder(quantize_audio_weights(synthetic_audio_dense(cfg, seed=0), cfg, device))
    gen = torch.Generator(device=device)
    gen.manual_seed(1)
    feats_in = torch.randn(NB * FRAMES, cfg.d_model, generator=gen, device=device).to(torch.bfloat16).float()
    h = feats_in.clone()
    enc.encoder_layers(h, [FRAMES * i for i in range(NB + 1)])
    out = enc.head(h)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(out).all())
    return enc, feats_in.cpu(), out


def test_c5_encoder_matches_oracle(c5_encoder):
    from torch2vk_amd.qwen3_asr.encoder import audio_tensor_shapes

    enc, feats_in, out = c5_encoder
    cfg = enc.config
    w = oasr.dense_from_packed({k: v.cpu().numpy() for k, v in enc.weights.packed.items()},
                               {k: v.cpu().numpy() for k, v in enc.weights.vectors.items()}, audio_tensor_shapes(cfg))
    got = out.cpu().numpy()
    for b in (0, NB - 1):
        rows = slice(b * FRAMES, (b + 1) * FRAMES)
        print(f"c5 encoder: oracle over utterance {b}", flush=True)
        h = oasr.encoder_layers_cpu(w, cfg, feats_in[rows].clone(), cu_seqlens=[0, FRAMES])
        ref = oasr.encoder_head_cpu(w, cfg, h).numpy()
        scale = float(np.abs(ref).max())
        err = float(np.abs(got[rows] - ref).max())
        print(f"c5 encoder utterance {b}: max-abs {err:.3e} of max |ref| {scale:.3e}", flush=True)
        # the tolerance of the 18-layer tower test (bf16 GEMM inputs, q/k/v and P against an fp32 oracle)
        assert_close(got[rows], ref, max_abs=5e-2 * scale, min_cos=0.999, what=f"utterance {b}")
        for r in (0, 103, 104, 777, FRAMES - 1):
            assert_close(got[rows][r], ref[r], max_abs=5e-2 * scale, min_cos=0.999, what=f"utterance {b} row {r}")


def test_c5_decoder_group_full_depth_matches_oracle(device, c5_encoder):
    from torch2vk_amd.qwen3.config import QWEN3_0_6B
    from torch2vk_amd.qwen3.model import Qwen3DecoderGroup
    from torch2vk_amd.qwen3.weights import matrix_shapes, synthetic_weights
    from torch2vk_amd.qwen3_asr.config import AUDIO_TOKEN_ID
    from torch2vk_amd.qwen3_asr.encoder import run_audio_inject

    _, _, feats = c5_encoder
    cfg = QWEN3_0_6B
    print("c5 decoder: 28-layer 0.6B weights", flush=True)
    w = synthetic_weights(cfg, device=device, seed=2)
    prefix, suffix = [151644, 8948, 198, 151669], [151670, 151645, 198]
    prompt = prefix + [AUDIO_TOKEN_ID] * FRAMES + suffix
    n = len(prompt)
    group = Qwen3DecoderGroup.create(w, NB, max_positions=n + NEW_TOKENS + 16, max_new_tokens=NEW_TOKENS + 8,
                                     device=device)
    for d in group.decoders:
        d.stop_on_eos = False
    ids = torch.tensor(prompt, device=device)
    audio_pos = torch.arange(len(prefix), len(prefix) + FRAMES, device=device)
    embs = []
    for b, d in enumerate(group.decoders):
        e = d.embed_tokens(ids)
        run_audio_inject(e, audio_pos, feats[b * FRAMES:(b + 1) * FRAMES])
        embs.append(e)
    group.prefill_chunked(embs, chunk=2048)
    prefill_h = [d.h.clone() for d in group.decoders]
    toks = group.finish(NEW_TOKENS)
    for b, d in enumerate(group.decoders):
        assert int(d.status.item()) == 0, f"sequence {b}: status {int(d.status.item()):#x}"
        assert len(toks[b]) == NEW_TOKENS
    print(f"c5 decoder tokens {toks}", flush=True)
    shape = Qwen3Shape(hidden=cfg.hidden, layers=cfg.layers, heads=cfg.heads, kv_heads=cfg.kv_heads,
                       head_dim=cfg.head_dim, mlp=cfg.mlp, vocab=cfg.vocab, rope_theta=cfg.rope_theta)
    dense = dense_weights({k: v.cpu().numpy() for k, v in w.packed.items()}, w.types,
                          {k: v.cpu().numpy() for k, v in w.norms.items()}, matrix_shapes(cfg))
    for b, d in enumerate(group.decoders):
        print(f"c5 decoder: oracle over sequence {b} ({n} prompt positions)", flush=True)
        stats = check_greedy_tokens(shape, dense, prompt, toks[b], prompt_embeds=embs[b].cpu(),
                                    kv_history=(d.k_cache, d.v_cache),
                                    gpu_logits=decoder_step_logits(d, prefill_h[b]), label=f"c5 sequence {b}")
        print(f"c5 sequence {b}: {stats}", flush=True)
