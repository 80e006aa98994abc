"""The reference-named operator surface on the GPU: each variant called by name with the reference's physical
weight types (Q4_K uint32 words, Q6_K / Q8_0 uint16 halfwords) against the CPU oracle, the row-count rule that
picks a GEMV or the matrix-core GEMM (src/torch2vk/export/shaders/linear_nobias_quantized.py:47-80), and
run_decode_layer over every layer of a small model against the decoder's fused path and the oracle's tokens."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from oracle import reference as R
from tests.conftest import assert_close

pytestmark = pytest.mark.gpu

_PHYS = {"q4_k": torch.uint32, "q6_k": torch.uint16, "q8_0": torch.uint16}


def _weight(wtype, n, k, seed, device):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((n, k)) * 0.03).astype(np.float32)
    packed = getattr(oracle, f"quantize_{wtype}")(w)
    wd = getattr(oracle, f"dequant_{wtype}")(packed, k)
    return torch.from_numpy(packed).to(device).view(_PHYS[wtype]), wd, rng


def _x(rng, m, k, device):
    x = R.bf16_round(rng.standard_normal((m, k)).astype(np.float32))
    return x, torch.from_numpy(x).to(device).to(torch.bfloat16)


@pytest.mark.parametrize("wtype", ["q4_k", "q6_k", "q8_0"])
def test_matvec_variants_by_name(device, wtype):
    from torch2vk_amd import variants as V
    from torch2vk_amd.runtime import RuntimeSession

    n, k = 96, 1024
    print(f"matvec variant {wtype} N={n} K={k}", flush=True)
    w, wd, rng = _weight(wtype, n, k, 5, device)
    x, xt = _x(rng, 1, k, device)
    ref = R.gemv_ref(x, wd)
    scale = np.abs(ref).max()
    rt = RuntimeSession(device, record=True)
    plain = {"q4_k": V.LINEAR_NOBIAS_Q4_K_MATVEC_F32, "q6_k": V.LINEAR_NOBIAS_Q6_K_MATVEC_F32,
             "q8_0": V.LINEAR_NOBIAS_Q8_0_MATVEC_F32}[wtype]
    out = torch.zeros(1, 1, n, device=device)
    plain(rt, x=xt.view(1, 1, k), weight=w, output=out)
    assert_close(out.view(1, n).cpu().numpy(), ref, max_abs=2e-4 * scale + 1e-6, min_cos=0.99999, what=plain.name)
    assert rt.records[-1].shader == plain.name
    if wtype != "q8_0":
        add = V.LINEAR_NOBIAS_Q4_K_MATVEC_ADD_F32 if wtype == "q4_k" else V.LINEAR_NOBIAS_Q6_K_MATVEC_ADD_F32
        res = rng.standard_normal((1, 1, n)).astype(np.float32)
        h = torch.from_numpy(res).to(device)
        add(rt, x=xt.view(1, 1, k), weight=w, residual=h, output=h)   # in place, as the decode layer runs it
        assert_close(h.view(1, n).cpu().numpy(), ref + res.reshape(1, n), max_abs=2e-4 * scale + 1e-5,
                     min_cos=0.99999, what=add.name)


@pytest.mark.parametrize("v_type", ["q4_k", "q6_k"])
def test_qkv_matvec_variants_by_name(device, v_type):
    from torch2vk_amd import variants as V
    from torch2vk_amd.runtime import RuntimeSession

    k = 1024
    wq, dq, rng = _weight("q4_k", 128, k, 1, device)
    wk, dk, _ = _weight("q4_k", 64, k, 2, device)
    wv, dv, _ = _weight(v_type, 64, k, 3, device)
    x, xt = _x(rng, 1, k, device)
    outs = [torch.zeros(1, 1, n, device=device) for n in (128, 64, 64)]
    var = V.LINEAR_NOBIAS_Q4_K_QKV_MATVEC_F32 if v_type == "q4_k" else V.LINEAR_NOBIAS_Q4_QK_Q6_V_MATVEC_F32
    print(f"{var.name}", flush=True)
    var(RuntimeSession(device), x=xt.view(1, 1, k), q_weight=wq, k_weight=wk, v_weight=wv, q_output=outs[0],
        k_output=outs[1], v_output=outs[2])
    for o, d, nm in zip(outs, (dq, dk, dv), "qkv"):
        ref = R.gemv_ref(x, d)
        assert_close(o.view(1, -1).cpu().numpy(), ref, max_abs=2e-4 * np.abs(ref).max() + 1e-6, min_cos=0.99999,
                     what=f"{var.name} {nm}")
    g = [torch.zeros(1, 1, 128, device=device, dtype=torch.bfloat16) for _ in range(2)]
    V.LINEAR_NOBIAS_Q4_K_QK_MATVEC_F32(RuntimeSession(device), x=xt.view(1, 1, k), q_weight=wq, k_weight=wq,
                                       q_output=g[0], k_output=g[1])
    assert torch.equal(g[0], g[1])
    ref = R.gemv_ref(x, dq)
    assert_close(g[0].float().view(1, -1).cpu().numpy(), ref, max_abs=1e-2 * np.abs(ref).max(), min_cos=0.9999,
                 what="qk matvec bf16")


@pytest.mark.parametrize("wtype", ["q4_k", "q6_k", "q8_0"])
@pytest.mark.parametrize("m", [1, 8, 9, 33])
def test_rows_pick_gemv_or_gemm(device, wtype, m):
    """M <= 8 rows: the GEMV once per row; above, or for a shape the GEMVs are not built for: the matrix-core
    GEMM.  Both through kernels.quantized_linear and through the named variants, against x . deq(W)^T in
    float64."""
    from torch2vk_amd import kernels
    from torch2vk_amd import variants as V
    from torch2vk_amd.runtime import RuntimeSession, weight_layout

    n, k = 80, 512
    print(f"quantized linear {wtype} M={m}", flush=True)
    w, wd, rng = _weight(wtype, n, k, 100 + m, device)
    x, xt = _x(rng, m, k, device)
    ref = R.gemv_ref(x, wd)
    gemv = m <= 8 and kernels.matvec_supported(wtype, k, n)   # Q6_K at K = 512 is not built: the GEMM runs
    assert gemv == (m <= 8 and wtype != "q6_k")
    if not gemv:
        # the GEMM rounds the dequantised weight tile to bf16 for the matrix cores: against x . bf16(deq W)^T
        # only the fp32 accumulation differs (the GEMVs keep the weights exact in fp32)
        ref = x.astype(np.float64) @ R.bf16_round(wd.astype(np.float32)).astype(np.float64).T
    tol = 2e-4 * np.abs(ref).max() + 1e-6 if gemv else 1e-5 * np.abs(ref).max() + 1e-6
    got = kernels.quantized_linear(xt, w.view(torch.uint8), wtype)
    assert got.dtype == torch.float32 and got.shape == (m, n)
    assert_close(got.cpu().numpy(), ref, max_abs=tol, min_cos=0.99999, what=f"quantized_linear {wtype} M={m}")
    res = rng.standard_normal((m, n)).astype(np.float32)
    h = torch.from_numpy(res).to(device)
    kernels.quantized_linear(xt, w.view(torch.uint8), wtype, out=h, residual=h)
    assert_close(h.cpu().numpy(), ref + res, max_abs=tol + 1e-5, min_cos=0.99999, what="with residual")

    rt = RuntimeSession(device, record=True)
    out = torch.zeros(1, m, n, device=device)
    V.run_linear_nobias_quantized(rt, x=xt.view(1, m, k), weight=w, output=out)
    picked = V.linear_nobias_quantized_variant(m, weight_layout(w, k))
    assert rt.records[-1].shader == picked.name
    assert ("matvec" in picked.name) == (m <= 8)
    assert_close(out.view(m, n).cpu().numpy(), ref, max_abs=tol, min_cos=0.99999, what=picked.name)


def test_norm_swiglu_embedding_variants(device):
    from torch2vk_amd import variants as V
    from torch2vk_amd.runtime import RuntimeSession

    rt = RuntimeSession(device)
    rng = np.random.default_rng(9)
    h = rng.standard_normal((1, 3, 512)).astype(np.float32)
    wn = (1 + 0.1 * rng.standard_normal(512)).astype(np.float32)
    out = torch.zeros(1, 3, 512, dtype=torch.bfloat16, device=device)
    V.RMS_NORM_MUL_F16_F32(rt, x=torch.from_numpy(h).to(device), weight=torch.from_numpy(wn).to(device), output=out)
    ref = R.rms_norm(h, wn)
    assert_close(out.float().cpu().numpy(), ref, max_abs=1e-2 * np.abs(ref).max(), min_cos=0.9999, what="rms_norm")

    g = rng.standard_normal((1, 2, 768)).astype(np.float32)
    u = rng.standard_normal((1, 2, 768)).astype(np.float32)
    act = torch.zeros(1, 2, 768, dtype=torch.bfloat16, device=device)
    V.SWIGLU_F16(rt, gate=torch.from_numpy(g).to(device), up=torch.from_numpy(u).to(device), output=act)
    ref = R.silu_mul(g, u)
    assert_close(act.float().cpu().numpy(), ref, max_abs=1e-2 * np.abs(ref).max(), min_cos=0.9999, what="swiglu")

    w, wd, _ = _weight("q4_k", 50, 512, 4, device)
    ids = torch.tensor([[3, 49, 0, 3]], dtype=torch.int64, device=device)
    emb = torch.zeros(1, 4, 512, device=device)
    V.EMBEDDING_Q4_K_F32(rt, weight=w, indices=ids, output=emb)
    np.testing.assert_array_equal(emb.view(4, 512).cpu().numpy(), wd[[3, 49, 0, 3]].astype(np.float32))


@pytest.mark.parametrize("pos_on_device", [False, True])
def test_sdpa_decode_cache_write_by_name(device, pos_on_device):
    """q / new_k already normalised and rotated: new_k / new_v land in row cache_position (bf16), the output is
    softmax(q K^T / sqrt(D)) V over rows 0..cache_position (sdpa_decode_cache_write_f32.py:104-168)."""
    from torch2vk_amd import variants as V
    from torch2vk_amd.runtime import RuntimeSession

    nh, nk, d, s, pos = 8, 2, 128, 64, 37
    print(f"sdpa decode pos={pos} device_pos={pos_on_device}", flush=True)
    rng = np.random.default_rng(17)
    kc = R.bf16_round(rng.standard_normal((1, s, nk, d)).astype(np.float32))
    vc = R.bf16_round(rng.standard_normal((1, s, nk, d)).astype(np.float32))
    q = rng.standard_normal((1, nh, 1, d)).astype(np.float32) * 0.2
    kn = rng.standard_normal((1, nk, 1, d)).astype(np.float32)
    vn = rng.standard_normal((1, 1, nk, d)).astype(np.float32)
    t = lambda a, dt=torch.float32: torch.from_numpy(np.ascontiguousarray(a)).to(device).to(dt)  # noqa: E731
    k_cache, v_cache = t(kc, torch.bfloat16), t(vc, torch.bfloat16)
    out = torch.zeros(1, nh, 1, d, dtype=torch.bfloat16, device=device)
    cp = torch.tensor([pos], dtype=torch.int32, device=device) if pos_on_device else pos
    V.SDPA_DECODE_CACHE_WRITE_F32(RuntimeSession(device), q=t(q), new_k=t(kn), new_v=t(vn), k_cache=k_cache,
                                  v_cache=v_cache, output=out, cache_position=cp)
    kc[0, pos] = R.bf16_round(kn[0, :, 0, :])
    vc[0, pos] = R.bf16_round(vn[0, 0])
    np.testing.assert_array_equal(k_cache.float().cpu().numpy(), kc)
    np.testing.assert_array_equal(v_cache.float().cpu().numpy(), vc)
    ref = R.attention_ref(q[0, :, 0, :][None], kc[0, :pos + 1], vc[0, :pos + 1])[0]
    assert_close(out.float().view(nh, d).cpu().numpy(), ref, max_abs=2 ** -7 * max(1.0, np.abs(ref).max()),
                 min_cos=0.9999, what="sdpa decode")


TINY = dict(hidden=256, layers=2, heads=4, kv_heads=2, head_dim=128, mlp=768, vocab=1024)


def _model(device, policy, cfg_kw, seed):
    from oracle.qwen3_check import dense_weights
    from oracle.reference import Qwen3Shape
    from torch2vk_amd.qwen3.config import Qwen3Config
    from torch2vk_amd.qwen3.weights import matrix_shapes, synthetic_weights

    cfg = Qwen3Config("variants", **cfg_kw, eos_token_ids=(cfg_kw["vocab"] - 1,))
    w = synthetic_weights(cfg, device=device, seed=seed, std=0.06, norm_std=0.1, policy=policy)
    dense = dense_weights({k: v.cpu().numpy() for k, v in w.packed.items()}, w.types,
                          {k: v.cpu().numpy() for k, v in w.norms.items()}, matrix_shapes(cfg))
    shape = Qwen3Shape(hidden=cfg.hidden, layers=cfg.layers, heads=cfg.heads, kv_heads=cfg.kv_heads,
                       head_dim=cfg.head_dim, mlp=cfg.mlp, vocab=cfg.vocab, rope_theta=cfg.rope_theta)
    return cfg, w, dense, shape


def test_run_decode_layer_matches_fused_path(device):
    """One step of every layer through the named variants equals the decoder's fused per-op step (RMSNorm in
    the GEMV prologues, SwiGLU in the gate|up epilogue) to bf16 rounding of the activations; KV rows match."""
    from torch2vk_amd.qwen3.dispatch import bind_model_tensors, run_decode_layer, run_decode_rope
    from torch2vk_amd.qwen3.model import Qwen3Decoder
    from torch2vk_amd.runtime import RuntimeSession

    cfg, w, _, _ = _model(device, "uniform", TINY, 31)
    dec = Qwen3Decoder(w, max_positions=64, max_new_tokens=8, persistent=False)
    dec.stop_on_eos = False
    dec.prefill(torch.tensor([4, 77, 901, 12, 5]))
    pos = int(dec.position.item())
    dec.run_decode_embed()
    h0, kc0, vc0 = dec.h.clone(), dec.k_cache.clone(), dec.v_cache.clone()
    for i in range(cfg.layers):
        dec.run_decode_layer(i)
    h_fused, kc_fused = dec.h.clone(), dec.k_cache.clone()
    dec.h.copy_(h0)
    dec.k_cache.copy_(kc0)
    dec.v_cache.copy_(vc0)
    rt = RuntimeSession(device, record=True)
    bind_model_tensors(dec)
    run_decode_rope(rt, cache_position=pos, rope_theta=cfg.rope_theta)
    for i in range(cfg.layers):
        run_decode_layer(rt, i, cache_position=pos)
    names = [r.shader for r in rt.records]
    # the reference's sequence (decode_layer.py:60-128) after the step's RoPE table
    assert names[:11] == ["rope_table_f32", "rms_norm_mul_f16_f32", "linear_nobias_q4_k_qkv_matvec_f32",
                          "rms_norm_rope_transpose_f16", "rms_norm_rope_transpose_f16",
                          "sdpa_decode_cache_write_f32", "linear_nobias_q4_k_matvec_add_f32",
                          "rms_norm_mul_f16_f32", "linear_nobias_q4_k_qk_matvec_f32", "swiglu_f16",
                          "linear_nobias_q4_k_matvec_add_f32"] and len(names) == 1 + 10 * cfg.layers
    scale = float(h_fused.abs().max())
    assert_close(dec.h.cpu().numpy(), h_fused.cpu().numpy(), max_abs=1e-2 * scale, min_cos=0.9999, what="h")
    # layer 0's new K row: the table-driven q/k norm + RoPE and the fused attention prologue share their
    # arithmetic (rope.h), and the RMSNorm + q|k|v GEMVs read the same bf16 input, so the row is bit-identical
    assert torch.equal(dec.k_cache[0, pos], kc_fused[0, pos])
    assert_close(dec.k_cache[:, pos].float().cpu().numpy(), kc_fused[:, pos].float().cpu().numpy(),
                 max_abs=3e-2, min_cos=0.9999, what="k row")
    assert torch.equal(dec.k_cache[:, :pos], kc_fused[:, :pos])


@pytest.mark.parametrize("policy,cfg_kw", [
    ("uniform", TINY),
    ("q4_k_m", dict(hidden=1024, layers=4, heads=8, kv_heads=2, head_dim=128, mlp=1024, vocab=1024)),
])
def test_variant_decode_matches_oracle(device, policy, cfg_kw):
    """Greedy decode where every layer runs as run_decode_layer(rt, i, cache_position=pos) and the embedding
    as EMBEDDING_Q4_K_F32 (Q4_K_M: the Q6_K v rows through LINEAR_NOBIAS_Q4_QK_Q6_V_MATVEC_F32 and Q6_K o/down
    through the Q6_K add variant) -- the oracle's tokens."""
    from oracle.qwen3_check import check_greedy_tokens, decoder_step_logits
    from torch2vk_amd import variants as V
    from torch2vk_amd.qwen3.dispatch import bind_model_tensors, run_decode_layer, run_decode_rope
    from torch2vk_amd.qwen3.model import Qwen3Decoder
    from torch2vk_amd.runtime import RuntimeSession

    cfg, w, dense, shape = _model(device, policy, cfg_kw, 41)
    dec = Qwen3Decoder(w, max_positions=64, max_new_tokens=16, persistent=False)
    rt = RuntimeSession(device, record=True)
    bind_model_tensors(dec)
    prompt = np.random.default_rng(2).integers(0, cfg.vocab, 6).tolist()
    n_new = 10
    print(f"variant decode {policy}: prompt {prompt}", flush=True)
    embed = w.packed["embed"]
    toks, cur = [], prompt[0]
    for step in range(len(prompt) + n_new - 1):
        dec.next_token.fill_(cur)
        if w.types["embed"] == "q4_k":
            V.EMBEDDING_Q4_K_F32(rt, weight=embed.view(torch.uint32), indices=dec.next_token,
                                 output=dec.h.view(1, 1, cfg.hidden))
        else:
            dec.run_decode_embed()
        run_decode_rope(rt, cache_position=step, rope_theta=cfg.rope_theta)
        for i in range(cfg.layers):
            run_decode_layer(rt, i, cache_position=step)
        dec.run_lm_head_select()
        nxt = int(dec.next_token.item())
        if step >= len(prompt) - 1:
            toks.append(nxt)
        cur = prompt[step + 1] if step + 1 < len(prompt) else nxt
    used = {r.shader for r in rt.records}
    if policy == "q4_k_m":
        assert {"linear_nobias_q4_qk_q6_v_matvec_f32", "linear_nobias_q6_k_matvec_add_f32"} <= used
    print(f"variant decode {policy}: {toks}", flush=True)
    print(check_greedy_tokens(shape, dense, prompt, toks, kv_history=(dec.k_cache, dec.v_cache),
                              gpu_logits=decoder_step_logits(dec), label=f"variants {policy}"))
