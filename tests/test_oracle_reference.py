"""Pins the oracle's reference math and CPU decoder against independent implementations (CPU only).

* attention: torch.nn.functional.scaled_dot_product_attention (GQA by head repeat);
* RMSNorm / SiLU: torch's own ops;
* the whole Qwen3 decoder (q/k-norm, rotate-half RoPE with theta 1e6, GQA,
  SwiGLU, pre-norm residuals, final norm, untied LM head): transformers'
  Qwen3ForCausalLM built from a local random-init config (no download).
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import reference as R


def test_argmax_ties_go_to_lowest_id():
    s = np.array([0.5, 2.0, -1.0, 2.0, 2.0, 1.9999])
    assert R.argmax_lowest(s) == 1
    assert R.argmax_lowest(np.array([3.0])) == 0


def test_rms_norm_and_silu_match_torch():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((5, 96)) * 3
    w = 1 + 0.1 * rng.standard_normal(96)
    ref = torch.nn.functional.rms_norm(torch.from_numpy(x), (96,), torch.from_numpy(w), eps=R.RMS_EPS).numpy()
    np.testing.assert_allclose(R.rms_norm(x, w), ref, rtol=1e-12, atol=1e-12)
    g, u = rng.standard_normal(50), rng.standard_normal(50)
    np.testing.assert_allclose(R.silu_mul(g, u), (torch.nn.functional.silu(torch.from_numpy(g)) * torch.from_numpy(u)).numpy(),
                               rtol=1e-12)


@pytest.mark.parametrize("causal", [None, 3])
def test_attention_matches_torch_sdpa(causal):
    rng = np.random.default_rng(2)
    t, nh, nk, s, d = 4, 8, 2, 11, 16
    q = rng.standard_normal((t, nh, d))
    k = rng.standard_normal((s, nk, d))
    v = rng.standard_normal((s, nk, d))
    got = R.attention_ref(q, k, v, causal_offset=causal)
    qt = torch.from_numpy(q).permute(1, 0, 2)[None]
    kt = torch.from_numpy(k).repeat_interleave(nh // nk, dim=1).permute(1, 0, 2)[None]
    vt = torch.from_numpy(v).repeat_interleave(nh // nk, dim=1).permute(1, 0, 2)[None]
    mask = None
    if causal is not None:
        mask = torch.from_numpy(np.arange(s)[None, :] <= (causal + np.arange(t))[:, None])
    ref = torch.nn.functional.scaled_dot_product_attention(qt, kt, vt, attn_mask=mask)[0].permute(1, 0, 2).numpy()
    np.testing.assert_allclose(got, ref, rtol=1e-10, atol=1e-10)


def test_rope_tables_match_closed_form():
    cos, sin = R.rope_cos_sin(np.array([0, 5, 4096]), 128, 1e6)
    assert cos.shape == (3, 128)
    np.testing.assert_allclose(cos[0], 1.0)
    np.testing.assert_allclose(sin[0], 0.0)
    # dims d and d + 64 share a frequency; frequency 0 is 1 rad per position
    np.testing.assert_allclose(cos[:, :64], cos[:, 64:])
    np.testing.assert_allclose(cos[1, 0], math.cos(5.0))
    np.testing.assert_allclose(sin[2, 63], math.sin(4096 * 1e6 ** (-126 / 128)))


def _hf_model(shape: R.Qwen3Shape, seed: int):
    from transformers import Qwen3Config, Qwen3ForCausalLM

    cfg = Qwen3Config(hidden_size=shape.hidden, intermediate_size=shape.mlp, num_hidden_layers=shape.layers,
                      num_attention_heads=shape.heads, num_key_value_heads=shape.kv_heads, head_dim=shape.head_dim,
                      vocab_size=shape.vocab, rms_norm_eps=R.RMS_EPS, tie_word_embeddings=False,
                      max_position_embeddings=512,
                      rope_parameters={"rope_type": "default", "rope_theta": shape.rope_theta})
    torch.manual_seed(seed)
    model = Qwen3ForCausalLM(cfg).eval().to(torch.float64)
    with torch.no_grad():
        for p in model.parameters():
            p.normal_(0, 0.05)
        for name, p in model.named_parameters():
            if "norm" in name:
                p.add_(1.0)
    return model


def _dense_from_hf(model, shape):
    sd = model.state_dict()
    w = {"embed": sd["model.embed_tokens.weight"], "lm_head": sd["lm_head.weight"], "norm": sd["model.norm.weight"]}
    names = {"q": "self_attn.q_proj", "k": "self_attn.k_proj", "v": "self_attn.v_proj", "o": "self_attn.o_proj",
             "gate": "mlp.gate_proj", "up": "mlp.up_proj", "down": "mlp.down_proj"}
    for i in range(shape.layers):
        for k, n in names.items():
            w[f"layers.{i}.{k}"] = sd[f"model.layers.{i}.{n}.weight"]
        w[f"layers.{i}.input_norm"] = sd[f"model.layers.{i}.input_layernorm.weight"]
        w[f"layers.{i}.post_norm"] = sd[f"model.layers.{i}.post_attention_layernorm.weight"]
        w[f"layers.{i}.q_norm"] = sd[f"model.layers.{i}.self_attn.q_norm.weight"]
        w[f"layers.{i}.k_norm"] = sd[f"model.layers.{i}.self_attn.k_norm.weight"]
    return w


def test_cpu_decoder_matches_transformers_qwen3():
    shape = R.Qwen3Shape(hidden=64, layers=2, heads=4, kv_heads=2, head_dim=32, mlp=96, vocab=120, rope_theta=1e6)
    hf = _hf_model(shape, seed=3)
    ours = R.Qwen3CpuModel(shape, _dense_from_hf(hf, shape), max_positions=32, dtype=torch.float64)
    tokens = torch.tensor([5, 17, 99, 3, 64, 2, 110])
    with torch.no_grad():
        ref = hf(tokens[None]).logits[0]
    # prefill the first 5 tokens at once, then two single-token decode steps.  Both sides run RMSNorm in
    # fp32 (as HF does) and the oracle's attention in fp32, so agreement is at the 1e-7 level; a wrong
    # RoPE convention, GQA mapping, norm placement or missing q/k-norm moves logits by O(0.1).
    h = ours.forward(tokens[:5], start=0)
    torch.testing.assert_close(ours.logits(h), ref[4], rtol=1e-4, atol=1e-6)
    for t in (5, 6):
        h = ours.forward(tokens[t:t + 1], start=t)
        torch.testing.assert_close(ours.logits(h), ref[t], rtol=1e-4, atol=1e-6)


def test_cpu_masked_forward_matches_transformers_qwen3():
    """The oracle's masked full-sequence pass (OmniVoice's LLM forward: an additive mask instead of causal,
    every position's final-normed hidden) against transformers given the same 4D additive mask; and with the
    causal mask written out additively it reproduces the oracle's own causal path exactly."""
    shape = R.Qwen3Shape(hidden=64, layers=2, heads=4, kv_heads=2, head_dim=32, mlp=96, vocab=120, rope_theta=1e6)
    hf = _hf_model(shape, seed=4)
    dense = _dense_from_hf(hf, shape)
    tokens = torch.tensor([5, 17, 99, 3, 64, 2, 110])
    t = tokens.numel()
    big = -1e30
    mask = torch.zeros(t, t, dtype=torch.float64)
    mask[:, 5:] = big                # two padded keys hidden from every query
    mask[5:, :] = 0.0                # ... except from the padded queries themselves
    mask[0, 3] = big                 # and one arbitrary hole
    with torch.no_grad():
        ref = hf.model(input_ids=tokens[None], attention_mask=mask[None, None]).last_hidden_state[0]
    ours = R.Qwen3CpuModel(shape, dense, max_positions=32, dtype=torch.float64)
    got = ours.forward(tokens, 0, mask=mask, all_positions=True)
    torch.testing.assert_close(got, ref, rtol=1e-4, atol=1e-6)
    # bidirectional: a later token changes an earlier position's output (it would not under causality)
    other = R.Qwen3CpuModel(shape, dense, max_positions=32, dtype=torch.float64)
    changed = other.forward(torch.tensor([5, 17, 99, 3, 64, 2, 111]), 0, mask=torch.zeros(t, t, dtype=torch.float64),
                            all_positions=True)
    same = R.Qwen3CpuModel(shape, dense, max_positions=32, dtype=torch.float64)
    base = same.forward(tokens, 0, mask=torch.zeros(t, t, dtype=torch.float64), all_positions=True)
    assert (changed[0] - base[0]).abs().max() > 1e-6
    causal = torch.triu(torch.full((t, t), big, dtype=torch.float64), diagonal=1)
    a = R.Qwen3CpuModel(shape, dense, max_positions=32, dtype=torch.float64)
    b = R.Qwen3CpuModel(shape, dense, max_positions=32, dtype=torch.float64)
    torch.testing.assert_close(a.forward(tokens, 0, mask=causal), b.forward(tokens, 0), rtol=0, atol=1e-12)
