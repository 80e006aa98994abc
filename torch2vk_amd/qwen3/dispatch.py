"""Qwen3 as the reference's exported-op surface: ``run_*(rt, ...)`` dispatch functions over bound model tensors.

Mirrors src/models/optimized_qwen3/dispatch/*.py and the step drivers of src/models/optimized_qwen3/run.py: every
function takes the runtime session, reads its tensors from ``model_tensors()`` and is a sequence of variant calls,
each checked against its contract by ``rt.dispatch``.

Decode (decode_embed.py, decode_layer.py:22-136, decode_norm.py; run.py:116-172):

    ROPE_TABLE_F32                              cos / sin of the cache position
    EMBEDDING_Q4_K_F32 (EMBEDDING_Q8_0_F32)     run_decode_embed
    per layer, run_decode_layer:
      RMS_NORM_MUL_F16_F32                      input RMSNorm
      LINEAR_NOBIAS_Q4_K_QKV_MATVEC_F32         q|k|v (LINEAR_NOBIAS_Q4_QK_Q6_V_MATVEC_F32 for a Q6_K v)
      RMS_NORM_ROPE_TRANSPOSE_F16 x 2           q/k RMSNorm + RoPE from the table
      SDPA_DECODE_CACHE_WRITE_F32               new K/V at cache_position + attention
      LINEAR_NOBIAS_Q{4,6}_K_MATVEC_ADD_F32     o_proj + residual
      RMS_NORM_MUL_F16_F32                      post-attention RMSNorm
      LINEAR_NOBIAS_Q4_K_QK_MATVEC_F32          gate|up
      SWIGLU_F16
      LINEAR_NOBIAS_Q{4,6}_K_MATVEC_ADD_F32     down + residual
    RMS_NORM_MUL_F16_F32                        run_decode_norm
    LM_HEAD_Q{6,4}_K_ARGMAX_PARTIAL_F16 + QWEN3_TOKEN_SELECT_REDUCE_CHUNKS_F32 + QWEN3_TOKEN_SELECT_REDUCE_F32
    QWEN3_TOKEN_STORE_EOS_F32

Prefill (embed_tokens.py, text_layer.py:232-271, text_norm.py; run.py:395-471): one full chunk of
``chunk`` tokens when the prompt is longer, then the tail, each with its own RoPE table, causal mask and mask
tile classes (FA_MASK_OPT_F16); per layer RMS_NORM_MUL_F32, three LLAMA_MATMUL GEMMs, RMS_NORM_ROPE_TOKEN_F32 (q)
and _TO_F16 (k), the token-major K/V cache writes (TRIPLE for the full chunk: the prompt cache, the chunk's
own flash cache and the decode cache; PAIR for the tail), LLAMA_FLASH_ATTN_F32_F16_F16, the o GEMM +
ADD_F32_PREFILL, RMS_NORM_MUL_F32, gate and up GEMMs, SWIGLU_F32, the down GEMM + ADD_F32_PREFILL; the tail's
last layer runs its MLP on the last token only (SLICE_LAST_TOKEN_F32_TO_F16, the GEMVs, ADD_F32_36).

Weights are the decoder's packed GGUF rows viewed as the reference's physical types (Q4_K uint32 words, Q6_K /
Q8_0 uint16 halfwords) without a copy; the KV caches are the decoder's.  Activations are bf16 (the reference's
fp16), the residual stream and the RoPE tables fp32.  Qwen3Decoder runs the same arithmetic with fewer launches
(fused prologues and epilogues) or, for decode, in one persistent launch.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from torch2vk_amd import variants as V
from torch2vk_amd.runtime import RuntimeSession


def _physical(w: torch.Tensor, wtype: str) -> torch.Tensor:
    """A packed GGUF row tensor (uint8 [N, row_bytes]) as the reference's word / halfword tensor."""
    return w.view(torch.uint32) if wtype == "q4_k" else w.view(torch.uint16)


# ------------------------------------------------------------------------------------- tensors --

@dataclass
class RopeTableTensors:
    """src/torch2vk/runtime/rope_table.py:25-29: fp32 cos / sin [1, T, D]."""
    cos: torch.Tensor
    sin: torch.Tensor


@dataclass
class DecodeEmbedTensors:
    """src/models/optimized_qwen3/tensors/decode_embed.py: the token id in, the residual row out."""
    p_weight: torch.Tensor               # embedding rows (Q4_K words or Q8_0 halfwords)
    input: torch.Tensor                  # int64 [1, 1], the decoder's next token
    embedding: torch.Tensor              # fp32 [1, 1, H], the decoder's residual stream


@dataclass
class DecodeNormTensors:
    """src/models/optimized_qwen3/tensors/decode_norm.py."""
    to: torch.Tensor                     # fp32 [1, 1, H], the residual stream after the last layer
    p_weight: torch.Tensor               # fp32 [H]
    mul_1: torch.Tensor                  # bf16 [1, 1, H], the LM head's input


@dataclass
class DecodeLayerTensors:
    """One decode layer's tensors in the reference's roles (src/models/optimized_qwen3/tensors/decode_layer.py)."""
    hidden: torch.Tensor                 # fp32 [1, 1, H], the residual stream (read and updated in place)
    normed: torch.Tensor                 # bf16 [1, 1, H]
    q: torch.Tensor                      # fp32 [1, 1, NQ]
    k: torch.Tensor                      # fp32 [1, 1, NKV]
    v: torch.Tensor                      # fp32 [1, 1, NKV]
    q_rot: torch.Tensor                  # fp32 [1, NH, 1, D]: q normalised and rotated (the reference's add_3)
    k_rot: torch.Tensor                  # fp32 [1, NK, 1, D] (add_4)
    attn: torch.Tensor                   # bf16 [1, NH, 1, D]
    gate: torch.Tensor                   # fp32 [1, 1, MLP]
    up: torch.Tensor                     # fp32 [1, 1, MLP]
    act: torch.Tensor                    # bf16 [1, 1, MLP]
    k_cache: torch.Tensor                # bf16 [1, S, NK, D]
    v_cache: torch.Tensor
    position_embeddings_0: torch.Tensor  # fp32 [1, 1, D], the decode RoPE table's cos
    position_embeddings_1: torch.Tensor  # its sin
    input_norm: torch.Tensor             # fp32 [H]
    post_norm: torch.Tensor
    q_norm: torch.Tensor                 # fp32 [D]
    k_norm: torch.Tensor
    q_weight: torch.Tensor               # uint32 Q4_K words
    k_weight: torch.Tensor
    v_weight: torch.Tensor               # uint32 Q4_K words or uint16 Q6_K halfwords
    o_weight: torch.Tensor
    gate_weight: torch.Tensor
    up_weight: torch.Tensor
    down_weight: torch.Tensor


@dataclass
class EmbedTokensTensors:
    """src/models/optimized_qwen3/tensors/embed_tokens.py: a prefill chunk's ids and embedding rows."""
    p_weight: torch.Tensor               # Q4_K words
    input: torch.Tensor                  # int64 [1, T]
    embedding: torch.Tensor              # fp32 [1, T, H], the chunk's residual stream


@dataclass
class TextLayerTensors:
    """One prefill layer over a chunk of T tokens (src/models/optimized_qwen3/tensors/text_layer.py), with the
    reference's names for the tensors its dispatch function reads.  The residual stream ``to`` is updated in
    place: the reference's add_5 / to_6 / add_7 are that buffer."""
    p_attn_q_proj_weight: torch.Tensor
    p_attn_k_proj_weight: torch.Tensor
    p_attn_v_proj_weight: torch.Tensor
    p_attn_o_proj_weight: torch.Tensor
    p_attn_q_norm_weight: torch.Tensor
    p_attn_k_norm_weight: torch.Tensor
    p_mlp_gate_proj_weight: torch.Tensor
    p_mlp_up_proj_weight: torch.Tensor
    p_mlp_down_proj_weight: torch.Tensor
    p_input_layernorm_weight: torch.Tensor
    p_post_attention_layernorm_weight: torch.Tensor
    position_embeddings_0: torch.Tensor  # fp32 [1, T, D]
    position_embeddings_1: torch.Tensor
    cache_position: torch.Tensor         # int64 [T]
    to: torch.Tensor                     # fp32 [1, T, H]
    mul_1: torch.Tensor                  # bf16 [1, T, H]
    linear: torch.Tensor                 # fp32 [1, T, NQ]
    linear_1: torch.Tensor               # fp32 [1, T, NKV]
    linear_2: torch.Tensor               # fp32 [1, T, NKV]
    to_2: torch.Tensor                   # linear as [1, T, NH, D]
    to_4: torch.Tensor                   # linear_1 as [1, T, NK, D]
    view_2: torch.Tensor                 # linear_2 as [1, T, NK, D]
    add_3: torch.Tensor                  # bf16 [1, T, NH, D], q normalised and rotated
    add_4: torch.Tensor                  # bf16 [1, T, NK, D], k normalised and rotated
    global_key_cache: torch.Tensor       # bf16 [1, S_attn, NK, D], the prompt's cache
    global_value_cache: torch.Tensor
    flash_key_cache: torch.Tensor        # the cache attention reads (the full chunk's own, else the prompt's)
    flash_value_cache: torch.Tensor
    decode_key_cache: torch.Tensor       # bf16 [1, S_max, NK, D], the decoder's
    decode_value_cache: torch.Tensor
    transpose_3: torch.Tensor            # bf16 [1, T, NH, D], attention output
    reshape: torch.Tensor                # transpose_3 as [1, T, NQ]
    linear_3: torch.Tensor               # fp32 [1, T, H]
    linear_4: torch.Tensor               # fp32 [1, T, MLP]
    linear_5: torch.Tensor
    mul_12: torch.Tensor                 # bf16 [1, T, MLP]
    linear_6: torch.Tensor               # fp32 [1, T, H]


@dataclass
class TextNormTensors:
    """src/models/optimized_qwen3/tensors/text_norm.py."""
    to: torch.Tensor                     # fp32 [1, 1, H], the last token's residual row
    p_weight: torch.Tensor
    mul_1: torch.Tensor                  # bf16 [1, 1, H]


@dataclass
class PrefillChunk:
    """One prefill chunk's tensors: its embedding, RoPE table, causal mask and tile classes, layers."""
    start: int
    embed: EmbedTokensTensors
    rope: RopeTableTensors
    causal_mask: torch.Tensor            # fp32 [T, S_attn], 0 or -inf
    mask_opt: torch.Tensor               # uint8 [1, ceil(T / 128), ceil(S_attn / 64)]
    layers: list[TextLayerTensors]


@dataclass
class ModelTensors:
    """The reference's model_tensors() (src/models/optimized_qwen3/tensors/model.py:60-370) over a decoder."""
    decode_rope: RopeTableTensors
    decode_embed: DecodeEmbedTensors
    decode_layers: list[DecodeLayerTensors]
    decode_norm: DecodeNormTensors
    lm_head_weight: torch.Tensor
    lm_head_partial_scores: torch.Tensor  # fp32 [G]
    lm_head_partial_tokens: torch.Tensor  # int32 [G] (the reference's uint32)
    lm_head_chunk_scores: torch.Tensor    # fp32 [ceil(G / 1024)]
    lm_head_chunk_tokens: torch.Tensor
    eos_token_ids: torch.Tensor           # int64 [E]
    next_token: torch.Tensor              # int64 [1, 1]
    done: torch.Tensor                    # int32 [1]
    generated_tokens: torch.Tensor        # int64 [1, max_new_tokens]
    generated_length: torch.Tensor        # int32 [1]
    stopped: torch.Tensor                 # int32 [1]
    embed_type: str
    lm_head_type: str
    prefill_full: PrefillChunk | None = None
    prefill_tail: PrefillChunk | None = None
    prefill_last_residual: torch.Tensor | None = None  # fp32 [1, 1, H] (the reference's is fp16)
    prefill_last_norm: torch.Tensor | None = None      # bf16 [1, 1, H]
    prefill_last_gate: torch.Tensor | None = None      # fp32 [1, 1, MLP]
    prefill_last_up: torch.Tensor | None = None
    prefill_last_gated: torch.Tensor | None = None     # bf16 [1, 1, MLP]
    prefill_last_down: torch.Tensor | None = None      # fp32 [1, 1, H]
    prefill_last_output: torch.Tensor | None = None    # fp32 [1, 1, H]
    text_norm: TextNormTensors | None = None
    decoder: object | None = None  # the Qwen3Decoder whose buffers these are


_MODEL: ModelTensors | None = None


def bind_model_tensors(decoder) -> ModelTensors:
    """Build the decode tensor sets over a Qwen3Decoder's weights, caches, residual stream and token state, and
    make them the ones the run_* functions use (the reference's model_tensors())."""
    global _MODEL
    c = decoder.config
    dev = decoder.device
    bf, f32 = torch.bfloat16, torch.float32
    w, n, t = decoder.weights.packed, decoder.weights.norms, decoder.types
    hidden = decoder.h.view(1, 1, c.hidden)
    rope = RopeTableTensors(torch.zeros(1, 1, c.head_dim, dtype=f32, device=dev),
                            torch.zeros(1, 1, c.head_dim, dtype=f32, device=dev))
    normed = torch.zeros(1, 1, c.hidden, dtype=bf, device=dev)
    q = torch.zeros(1, 1, c.q_dim, dtype=f32, device=dev)
    k = torch.zeros(1, 1, c.kv_dim, dtype=f32, device=dev)
    v = torch.zeros(1, 1, c.kv_dim, dtype=f32, device=dev)
    q_rot = torch.zeros(1, c.heads, 1, c.head_dim, dtype=f32, device=dev)
    k_rot = torch.zeros(1, c.kv_heads, 1, c.head_dim, dtype=f32, device=dev)
    attn = torch.zeros(1, c.heads, 1, c.head_dim, dtype=bf, device=dev)
    gate = torch.zeros(1, 1, c.mlp, dtype=f32, device=dev)
    up = torch.zeros(1, 1, c.mlp, dtype=f32, device=dev)
    act = torch.zeros(1, 1, c.mlp, dtype=bf, device=dev)
    layers = []
    for i in range(c.layers):
        p = f"layers.{i}."
        lw = {nm: _physical(w[p + nm], t[p + nm]) for nm in ("q", "k", "v", "o", "gate", "up", "down")}
        layers.append(DecodeLayerTensors(
            hidden=hidden, normed=normed, q=q, k=k, v=v, q_rot=q_rot, k_rot=k_rot, attn=attn, gate=gate, up=up,
            act=act, k_cache=decoder.k_cache[i].unsqueeze(0), v_cache=decoder.v_cache[i].unsqueeze(0),
            position_embeddings_0=rope.cos, position_embeddings_1=rope.sin,
            input_norm=n[p + "input_norm"], post_norm=n[p + "post_norm"], q_norm=n[p + "q_norm"],
            k_norm=n[p + "k_norm"], q_weight=lw["q"], k_weight=lw["k"], v_weight=lw["v"], o_weight=lw["o"],
            gate_weight=lw["gate"], up_weight=lw["up"], down_weight=lw["down"]))
    g = int(decoder.partial_scores.numel())
    chunks = -(-g // 1024)
    _MODEL = ModelTensors(
        decode_rope=rope,
        decode_embed=DecodeEmbedTensors(_physical(w["embed"], t["embed"]), decoder.next_token, hidden),
        decode_layers=layers,
        decode_norm=DecodeNormTensors(hidden, n["norm"], torch.zeros(1, 1, c.hidden, dtype=bf, device=dev)),
        lm_head_weight=_physical(w["lm_head"], t["lm_head"]),
        lm_head_partial_scores=decoder.partial_scores, lm_head_partial_tokens=decoder.partial_tokens,
        lm_head_chunk_scores=torch.zeros(chunks, dtype=f32, device=dev),
        lm_head_chunk_tokens=torch.zeros(chunks, dtype=torch.int32, device=dev),
        eos_token_ids=decoder.eos, next_token=decoder.next_token, done=decoder.done,
        generated_tokens=decoder.generated.view(1, -1), generated_length=decoder.length, stopped=decoder.stopped,
        embed_type=t["embed"], lm_head_type=t["lm_head"], decoder=decoder)
    return _MODEL


def model_tensors() -> ModelTensors:
    if _MODEL is None:
        raise RuntimeError("no model tensors bound: call bind_model_tensors(decoder) first")
    return _MODEL


def _causal_mask(chunk_start: int, chunk_length: int, attention_length: int, device) -> torch.Tensor:
    """fp32 [chunk_length, attention_length]: row r sees keys 0 .. chunk_start + r (run.py:270-274)."""
    keys = torch.arange(attention_length, device=device)
    rows = torch.arange(chunk_length, device=device)
    hidden = keys[None, :] > (chunk_start + rows)[:, None]
    return torch.zeros(chunk_length, attention_length, dtype=torch.float32, device=device).masked_fill_(
        hidden, float("-inf"))


def bind_prefill_tensors(prompt_ids: torch.Tensor, *, chunk: int = 512) -> ModelTensors:
    """Add a prompt's prefill tensors to the bound model (the reference's create_model_tensors for a prompt
    length, src/models/optimized_qwen3/tensors/model.py:75-250 with run.py:281-360): a full chunk of ``chunk``
    tokens when the prompt is longer, then the tail; the prompt's K/V caches of round_up(length, 64) positions,
    the full chunk's own flash caches, and the decoder's caches as the decode caches."""
    m = model_tensors()
    dec = m.decoder
    c = dec.config
    dev = dec.device
    bf, f32 = torch.bfloat16, torch.float32
    ids = prompt_ids.to(device=dev, dtype=torch.int64).reshape(1, -1)
    total = int(ids.shape[1])
    if total == 0:
        raise ValueError("empty prompt")
    if chunk <= 0:
        raise ValueError("chunk must be positive")
    full = chunk if total > chunk else 0
    s_attn = -(-total // 64) * 64
    if s_attn > dec.max_positions:
        raise ValueError(f"prompt of {total} needs {s_attn} cache positions, the decoder has {dec.max_positions}")
    w, n, t = dec.weights.packed, dec.weights.norms, dec.types
    kv_shape = (1, s_attn, c.kv_heads, c.head_dim)
    global_k = [torch.zeros(kv_shape, dtype=bf, device=dev) for _ in range(c.layers)]
    global_v = [torch.zeros(kv_shape, dtype=bf, device=dev) for _ in range(c.layers)]

    def make_chunk(start: int, length: int, attention_length: int, own_flash: bool) -> PrefillChunk:
        rope = RopeTableTensors(torch.zeros(1, length, c.head_dim, dtype=f32, device=dev),
                                torch.zeros(1, length, c.head_dim, dtype=f32, device=dev))
        mask = _causal_mask(start, length, attention_length, dev)
        mask_opt = torch.zeros(1, -(-length // 128), -(-attention_length // 64), dtype=torch.uint8, device=dev)
        hidden = torch.zeros(1, length, c.hidden, dtype=f32, device=dev)
        embed = EmbedTokensTensors(_physical(w["embed"], t["embed"]), ids[:, start:start + length].contiguous(),
                                   hidden)
        pos = torch.arange(start, start + length, dtype=torch.int64, device=dev)
        q = torch.zeros(1, length, c.q_dim, dtype=f32, device=dev)
        k = torch.zeros(1, length, c.kv_dim, dtype=f32, device=dev)
        v = torch.zeros(1, length, c.kv_dim, dtype=f32, device=dev)
        attn = torch.zeros(1, length, c.heads, c.head_dim, dtype=bf, device=dev)
        shared = dict(
            position_embeddings_0=rope.cos, position_embeddings_1=rope.sin, cache_position=pos, to=hidden,
            mul_1=torch.zeros(1, length, c.hidden, dtype=bf, device=dev), linear=q, linear_1=k, linear_2=v,
            to_2=q.view(1, length, c.heads, c.head_dim), to_4=k.view(1, length, c.kv_heads, c.head_dim),
            view_2=v.view(1, length, c.kv_heads, c.head_dim),
            add_3=torch.zeros(1, length, c.heads, c.head_dim, dtype=bf, device=dev),
            add_4=torch.zeros(1, length, c.kv_heads, c.head_dim, dtype=bf, device=dev),
            transpose_3=attn, reshape=attn.view(1, length, c.q_dim),
            linear_3=torch.zeros(1, length, c.hidden, dtype=f32, device=dev),
            linear_4=torch.zeros(1, length, c.mlp, dtype=f32, device=dev),
            linear_5=torch.zeros(1, length, c.mlp, dtype=f32, device=dev),
            mul_12=torch.zeros(1, length, c.mlp, dtype=bf, device=dev),
            linear_6=torch.zeros(1, length, c.hidden, dtype=f32, device=dev))
        layers = []
        for i in range(c.layers):
            p = f"layers.{i}."
            if own_flash:
                fk = torch.zeros(1, attention_length, c.kv_heads, c.head_dim, dtype=bf, device=dev)
                fv = torch.zeros_like(fk)
            else:
                fk, fv = global_k[i], global_v[i]
            layers.append(TextLayerTensors(
                p_attn_q_proj_weight=_physical(w[p + "q"], t[p + "q"]),
                p_attn_k_proj_weight=_physical(w[p + "k"], t[p + "k"]),
                p_attn_v_proj_weight=_physical(w[p + "v"], t[p + "v"]),
                p_attn_o_proj_weight=_physical(w[p + "o"], t[p + "o"]),
                p_attn_q_norm_weight=n[p + "q_norm"], p_attn_k_norm_weight=n[p + "k_norm"],
                p_mlp_gate_proj_weight=_physical(w[p + "gate"], t[p + "gate"]),
                p_mlp_up_proj_weight=_physical(w[p + "up"], t[p + "up"]),
                p_mlp_down_proj_weight=_physical(w[p + "down"], t[p + "down"]),
                p_input_layernorm_weight=n[p + "input_norm"], p_post_attention_layernorm_weight=n[p + "post_norm"],
                global_key_cache=global_k[i], global_value_cache=global_v[i], flash_key_cache=fk,
                flash_value_cache=fv, decode_key_cache=dec.k_cache[i].unsqueeze(0),
                decode_value_cache=dec.v_cache[i].unsqueeze(0), **shared))
        return PrefillChunk(start, embed, rope, mask, mask_opt, layers)

    m.prefill_full = make_chunk(0, full, full, True) if full else None
    m.prefill_tail = make_chunk(full, total - full, s_attn, False)
    m.prefill_last_residual = torch.zeros(1, 1, c.hidden, dtype=f32, device=dev)
    m.prefill_last_norm = torch.zeros(1, 1, c.hidden, dtype=bf, device=dev)
    m.prefill_last_gate = torch.zeros(1, 1, c.mlp, dtype=f32, device=dev)
    m.prefill_last_up = torch.zeros(1, 1, c.mlp, dtype=f32, device=dev)
    m.prefill_last_gated = torch.zeros(1, 1, c.mlp, dtype=bf, device=dev)
    m.prefill_last_down = torch.zeros(1, 1, c.hidden, dtype=f32, device=dev)
    m.prefill_last_output = torch.zeros(1, 1, c.hidden, dtype=f32, device=dev)
    m.text_norm = TextNormTensors(m.prefill_last_output, n["norm"], torch.zeros(1, 1, c.hidden, dtype=bf, device=dev))
    return m


# ------------------------------------------------------------------------------------ decode --

def _linear_q4_or_q6_add(rt: RuntimeSession, *, x: torch.Tensor, weight: torch.Tensor, residual: torch.Tensor,
                         output: torch.Tensor) -> None:
    """decode_layer.py:22-35: the Q6_K variant for halfword weights, else Q4_K."""
    if weight.dtype == torch.uint16:
        V.LINEAR_NOBIAS_Q6_K_MATVEC_ADD_F32(rt, x=x, weight=weight, residual=residual, output=output)
        return
    V.LINEAR_NOBIAS_Q4_K_MATVEC_ADD_F32(rt, x=x, weight=weight, residual=residual, output=output)


def _attn_qkv(rt: RuntimeSession, t: DecodeLayerTensors) -> None:
    """decode_layer.py:38-57."""
    variant = V.LINEAR_NOBIAS_Q4_QK_Q6_V_MATVEC_F32 if t.v_weight.dtype == torch.uint16 \
        else V.LINEAR_NOBIAS_Q4_K_QKV_MATVEC_F32
    variant(rt, x=t.normed, q_weight=t.q_weight, k_weight=t.k_weight, v_weight=t.v_weight, q_output=t.q,
            k_output=t.k, v_output=t.v)


def _run_decode_layer_with_tensors(rt: RuntimeSession, t: DecodeLayerTensors, *, cache_position) -> None:
    """decode_layer.py:60-128."""
    nh, d = t.attn.shape[1], t.attn.shape[3]
    nk = t.k_cache.shape[2]
    V.RMS_NORM_MUL_F16_F32(rt, x=t.hidden, weight=t.input_norm, output=t.normed)
    _attn_qkv(rt, t)
    V.RMS_NORM_ROPE_TRANSPOSE_F16(rt, x=t.q.view(1, 1, nh, d), weight=t.q_norm, cos=t.position_embeddings_0,
                                  sin=t.position_embeddings_1, output=t.q_rot)
    V.RMS_NORM_ROPE_TRANSPOSE_F16(rt, x=t.k.view(1, 1, nk, d), weight=t.k_norm, cos=t.position_embeddings_0,
                                  sin=t.position_embeddings_1, output=t.k_rot)
    V.SDPA_DECODE_CACHE_WRITE_F32(rt, q=t.q_rot, new_k=t.k_rot, new_v=t.v.view(1, 1, nk, d), k_cache=t.k_cache,
                                  v_cache=t.v_cache, cache_position=cache_position, output=t.attn)
    _linear_q4_or_q6_add(rt, x=t.attn.view(1, 1, nh * d), weight=t.o_weight, residual=t.hidden, output=t.hidden)
    V.RMS_NORM_MUL_F16_F32(rt, x=t.hidden, weight=t.post_norm, output=t.normed)
    V.LINEAR_NOBIAS_Q4_K_QK_MATVEC_F32(rt, x=t.normed, q_weight=t.gate_weight, k_weight=t.up_weight,
                                       q_output=t.gate, k_output=t.up)
    V.SWIGLU_F16(rt, gate=t.gate, up=t.up, output=t.act)
    _linear_q4_or_q6_add(rt, x=t.act, weight=t.down_weight, residual=t.hidden, output=t.hidden)


def run_decode_layer(rt: RuntimeSession, layer_idx: int, *, cache_position) -> None:
    """One decoder layer at ``cache_position`` (an int, or a one-element int32 device tensor) with the decode
    RoPE table as ROPE_TABLE_F32 last filled it (src/models/optimized_qwen3/dispatch/decode_layer.py:131-136)."""
    _run_decode_layer_with_tensors(rt, model_tensors().decode_layers[layer_idx], cache_position=cache_position)


def run_decode_rope(rt: RuntimeSession, *, cache_position, rope_theta: float) -> None:
    """The decode step's ROPE_TABLE_F32 (run.py:150-156)."""
    m = model_tensors()
    V.ROPE_TABLE_F32(rt, start_position=cache_position, theta=rope_theta, cos=m.decode_rope.cos, sin=m.decode_rope.sin)


def run_decode_embed(rt: RuntimeSession) -> None:
    """The next token's embedding row into the residual stream (src/models/optimized_qwen3/dispatch/
    decode_embed.py:14-19)."""
    m = model_tensors()
    e = m.decode_embed
    variant = V.EMBEDDING_Q8_0_F32 if m.embed_type == "q8_0" else V.EMBEDDING_Q4_K_F32
    variant(rt, weight=e.p_weight, indices=e.input, output=e.embedding)


def run_decode_norm(rt: RuntimeSession) -> None:
    """Final RMSNorm of the residual stream (src/models/optimized_qwen3/dispatch/decode_norm.py:14-19)."""
    t = model_tensors().decode_norm
    V.RMS_NORM_MUL_F16_F32(rt, x=t.to, weight=t.p_weight, output=t.mul_1)


def run_lm_head_select(rt: RuntimeSession, *, x: torch.Tensor) -> None:
    """LM head partial argmax, the chunk reduce and the final select with the EOS flag
    (_run_lm_head_select, src/models/optimized_qwen3/run.py:116-139)."""
    m = model_tensors()
    head = V.LM_HEAD_Q6_K_ARGMAX_PARTIAL_F16 if m.lm_head_type == "q6_k" else V.LM_HEAD_Q4_K_ARGMAX_PARTIAL_F16
    head(rt, x=x, weight=m.lm_head_weight, partial_scores=m.lm_head_partial_scores,
         partial_tokens=m.lm_head_partial_tokens)
    V.QWEN3_TOKEN_SELECT_REDUCE_CHUNKS_F32(rt, scores=m.lm_head_partial_scores, tokens=m.lm_head_partial_tokens,
                                           chunk_scores=m.lm_head_chunk_scores, chunk_tokens=m.lm_head_chunk_tokens)
    V.QWEN3_TOKEN_SELECT_REDUCE_F32(rt, partial_scores=m.lm_head_chunk_scores, partial_tokens=m.lm_head_chunk_tokens,
                                    eos_token_ids=m.eos_token_ids, next_token=m.next_token, done=m.done)


def run_token_store(rt: RuntimeSession, *, token_index) -> None:
    """QWEN3_TOKEN_STORE_EOS_F32 of the selected token at ``token_index`` (run.py:162-170, :457-466)."""
    m = model_tensors()
    V.QWEN3_TOKEN_STORE_EOS_F32(rt, next_token=m.next_token, token_index=token_index, done=m.done,
                                generated_tokens=m.generated_tokens, generated_length=m.generated_length,
                                stopped=m.stopped)


def run_decode_step(rt: RuntimeSession, *, cache_position: int, rope_theta: float, step: int) -> int:
    """One greedy decode step (_run_decode_step, src/models/optimized_qwen3/run.py:142-172): RoPE table, embed,
    every layer, final norm, LM head + select, token store at index step + 1; returns the selected token (a
    host read, as the reference's step does)."""
    m = model_tensors()
    run_decode_rope(rt, cache_position=cache_position, rope_theta=rope_theta)
    run_decode_embed(rt)
    for layer_idx in range(len(m.decode_layers)):
        run_decode_layer(rt, layer_idx, cache_position=cache_position)
    run_decode_norm(rt)
    run_lm_head_select(rt, x=m.decode_norm.mul_1)
    run_token_store(rt, token_index=step + 1)
    return int(m.next_token.view(-1)[0].item())


# ----------------------------------------------------------------------------------- prefill --

def _run_embed_tokens_with_tensors(rt: RuntimeSession, t: EmbedTokensTensors) -> None:
    V.EMBEDDING_Q4_K_ACT_F32(rt, weight=t.p_weight, indices=t.input, output=t.embedding)


def run_prefill_full_embed(rt: RuntimeSession) -> None:
    """src/models/optimized_qwen3/dispatch/embed_tokens.py:15-16."""
    _run_embed_tokens_with_tensors(rt, _chunk("full").embed)


def run_prefill_tail_embed(rt: RuntimeSession) -> None:
    """src/models/optimized_qwen3/dispatch/embed_tokens.py:19-20."""
    _run_embed_tokens_with_tensors(rt, _chunk("tail").embed)


def _chunk(which: str) -> PrefillChunk:
    m = model_tensors()
    ch = m.prefill_full if which == "full" else m.prefill_tail
    if ch is None:
        raise RuntimeError(f"no prefill {which} chunk bound: call bind_prefill_tensors(prompt_ids) first")
    return ch


def _llama_matmul(rt: RuntimeSession, *, x: torch.Tensor, weight: torch.Tensor, output: torch.Tensor) -> None:
    """text_layer.py:48-71: the Q6_K GEMM for halfword weights, else Q4_K; the _M tile at <= 320 tokens."""
    small = x.shape[0] * x.shape[1] <= 320
    if weight.dtype == torch.uint16:
        variant = V.LLAMA_MATMUL_Q6_K_F32_M if small else V.LLAMA_MATMUL_Q6_K_F32_L
    else:
        variant = V.LLAMA_MATMUL_Q4_K_F32_M if small else V.LLAMA_MATMUL_Q4_K_F32_L
    variant(rt, x=x, weight=weight, output=output)


def _linear_q4_or_q6_matvec(rt: RuntimeSession, *, x: torch.Tensor, weight: torch.Tensor,
                            output: torch.Tensor) -> None:
    """text_layer.py:80-84."""
    if weight.dtype == torch.uint16:
        V.LINEAR_NOBIAS_Q6_K_MATVEC_F32(rt, x=x, weight=weight, output=output)
        return
    V.LINEAR_NOBIAS_Q4_K_MATVEC_F32(rt, x=x, weight=weight, output=output)


def _attn_prologue(rt: RuntimeSession, t: TextLayerTensors, ch: PrefillChunk) -> None:
    """RMSNorm, q|k|v GEMMs, q/k norm + RoPE, the K/V cache writes and flash attention (text_layer.py:87-184)."""
    V.RMS_NORM_MUL_F32(rt, x=t.to, weight=t.p_input_layernorm_weight, output=t.mul_1)
    _llama_matmul(rt, x=t.mul_1, weight=t.p_attn_q_proj_weight, output=t.linear)
    _llama_matmul(rt, x=t.mul_1, weight=t.p_attn_k_proj_weight, output=t.linear_1)
    _llama_matmul(rt, x=t.mul_1, weight=t.p_attn_v_proj_weight, output=t.linear_2)
    V.RMS_NORM_ROPE_TOKEN_F32(rt, x=t.to_2, weight=t.p_attn_q_norm_weight, cos=t.position_embeddings_0,
                              sin=t.position_embeddings_1, output=t.add_3)
    V.RMS_NORM_ROPE_TOKEN_F32_TO_F16(rt, x=t.to_4, weight=t.p_attn_k_norm_weight, cos=t.position_embeddings_0,
                                     sin=t.position_embeddings_1, output=t.add_4)
    if t.flash_key_cache is not t.global_key_cache:
        V.TOKEN_MAJOR_KV_CACHE_WRITE_F16_TRIPLE(rt, cache_a=t.global_key_cache, cache_b=t.flash_key_cache,
                                                cache_c=t.decode_key_cache, cache_position=t.cache_position,
                                                src=t.add_4)
        V.TOKEN_MAJOR_VALUE_CACHE_WRITE_F32_TO_F16_TRIPLE(rt, cache_a=t.global_value_cache,
                                                          cache_b=t.flash_value_cache, cache_c=t.decode_value_cache,
                                                          cache_position=t.cache_position, src=t.view_2)
    else:
        V.TOKEN_MAJOR_KV_CACHE_WRITE_F16_PAIR(rt, cache_a=t.global_key_cache, cache_b=t.decode_key_cache,
                                              cache_position=t.cache_position, src=t.add_4)
        V.TOKEN_MAJOR_VALUE_CACHE_WRITE_F32_TO_F16_PAIR(rt, cache_a=t.global_value_cache, cache_b=t.decode_value_cache,
                                                        cache_position=t.cache_position, src=t.view_2)
    V.LLAMA_FLASH_ATTN_F32_F16_F16(rt, q=t.add_3, k=t.flash_key_cache, v=t.flash_value_cache, mask=ch.causal_mask,
                                   sink=t.add_3, output=t.transpose_3, mask_opt=ch.mask_opt)
    _llama_matmul(rt, x=t.reshape, weight=t.p_attn_o_proj_weight, output=t.linear_3)
    V.ADD_F32_PREFILL(rt, x=t.to, y=t.linear_3, output=t.to)


def _run_text_layer_with_tensors(rt: RuntimeSession, t: TextLayerTensors, ch: PrefillChunk) -> None:
    """text_layer.py:187-219."""
    _attn_prologue(rt, t, ch)
    V.RMS_NORM_MUL_F32(rt, x=t.to, weight=t.p_post_attention_layernorm_weight, output=t.mul_1)
    _llama_matmul(rt, x=t.mul_1, weight=t.p_mlp_gate_proj_weight, output=t.linear_4)
    _llama_matmul(rt, x=t.mul_1, weight=t.p_mlp_up_proj_weight, output=t.linear_5)
    V.SWIGLU_F32(rt, gate=t.linear_4, up=t.linear_5, output=t.mul_12)
    _llama_matmul(rt, x=t.mul_12, weight=t.p_mlp_down_proj_weight, output=t.linear_6)
    V.ADD_F32_PREFILL(rt, x=t.to, y=t.linear_6, output=t.to)


def _run_text_last_layer_tail_with_tensors(rt: RuntimeSession, t: TextLayerTensors, ch: PrefillChunk) -> None:
    """text_layer.py:222-263: attention over the chunk, then the MLP on the last token only."""
    m = model_tensors()
    _attn_prologue(rt, t, ch)
    V.SLICE_LAST_TOKEN_F32_TO_F16(rt, x=t.to, output=m.prefill_last_residual)
    V.RMS_NORM_MUL_F16_F32(rt, x=m.prefill_last_residual, weight=t.p_post_attention_layernorm_weight,
                           output=m.prefill_last_norm)
    V.LINEAR_NOBIAS_Q4_K_QK_MATVEC_F32(rt, x=m.prefill_last_norm, q_weight=t.p_mlp_gate_proj_weight,
                                       k_weight=t.p_mlp_up_proj_weight, q_output=m.prefill_last_gate,
                                       k_output=m.prefill_last_up)
    V.SWIGLU_F16(rt, gate=m.prefill_last_gate, up=m.prefill_last_up, output=m.prefill_last_gated)
    _linear_q4_or_q6_matvec(rt, x=m.prefill_last_gated, weight=t.p_mlp_down_proj_weight, output=m.prefill_last_down)
    V.ADD_F32_36(rt, x=m.prefill_last_residual, y=m.prefill_last_down, output=m.prefill_last_output)


def run_prefill_full_layer(rt: RuntimeSession, layer_idx: int) -> None:
    """src/models/optimized_qwen3/dispatch/text_layer.py:232-239."""
    ch = _chunk("full")
    _run_text_layer_with_tensors(rt, ch.layers[layer_idx], ch)


def run_prefill_tail_layer(rt: RuntimeSession, layer_idx: int) -> None:
    """src/models/optimized_qwen3/dispatch/text_layer.py:242-249."""
    ch = _chunk("tail")
    _run_text_layer_with_tensors(rt, ch.layers[layer_idx], ch)


def run_prefill_tail_last_layer_tail(rt: RuntimeSession) -> None:
    """src/models/optimized_qwen3/dispatch/text_layer.py:252-259."""
    ch = _chunk("tail")
    _run_text_last_layer_tail_with_tensors(rt, ch.layers[-1], ch)


def run_prefill_full_mask_opt(rt: RuntimeSession) -> None:
    """src/models/optimized_qwen3/dispatch/text_layer.py:262-267."""
    ch = _chunk("full")
    V.FA_MASK_OPT_F16(rt, mask=ch.causal_mask, output=ch.mask_opt)


def run_prefill_tail_mask_opt(rt: RuntimeSession) -> None:
    """src/models/optimized_qwen3/dispatch/text_layer.py:270-275."""
    ch = _chunk("tail")
    V.FA_MASK_OPT_F16(rt, mask=ch.causal_mask, output=ch.mask_opt)


def run_text_norm(rt: RuntimeSession) -> None:
    """Final RMSNorm of the prompt's last token (src/models/optimized_qwen3/dispatch/text_norm.py:14-19)."""
    t = model_tensors().text_norm
    if t is None:
        raise RuntimeError("no prefill bound: call bind_prefill_tensors(prompt_ids) first")
    V.RMS_NORM_MUL_F16_F32(rt, x=t.to, weight=t.p_weight, output=t.mul_1)


def run_prefill(rt: RuntimeSession, *, rope_theta: float) -> int:
    """The bound prompt's prefill as the reference's driver runs it (src/models/optimized_qwen3/run.py:395-471):
    the full chunk (RoPE table, embed, mask tiles, every layer), then the tail (its RoPE table, embed, mask
    tiles, every layer but the last, the last layer's tail), the final norm, LM head + select and the first
    token's store at index 0; returns that token (a host read)."""
    m = model_tensors()
    if m.prefill_full is not None:
        ch = m.prefill_full
        V.ROPE_TABLE_F32(rt, start_position=ch.start, theta=rope_theta, cos=ch.rope.cos, sin=ch.rope.sin)
        run_prefill_full_embed(rt)
        run_prefill_full_mask_opt(rt)
        for layer_idx in range(len(ch.layers)):
            run_prefill_full_layer(rt, layer_idx)
        # the tail continues from the full chunk's residual rows only through the caches
    ch = _chunk("tail")
    V.ROPE_TABLE_F32(rt, start_position=ch.start, theta=rope_theta, cos=ch.rope.cos, sin=ch.rope.sin)
    run_prefill_tail_embed(rt)
    run_prefill_tail_mask_opt(rt)
    for layer_idx in range(len(ch.layers) - 1):
        run_prefill_tail_layer(rt, layer_idx)
    run_prefill_tail_last_layer_tail(rt)
    run_text_norm(rt)
    run_lm_head_select(rt, x=m.text_norm.mul_1)
    run_token_store(rt, token_index=0)
    return int(m.next_token.view(-1)[0].item())


# ------------------------------------------------------- the exported (un-optimized) prefill names --
# src/models/quantized_qwen3/export.py:254-315 exports the same modules as three functions over the whole prompt
# (no chunking): embed_tokens, one decoder layer, the final norm of every position.  Here they run the
# optimized path's kernels over a prompt bound as one chunk (bind_prefill_tensors(prompt_ids, chunk=len)).

def _whole_prompt() -> PrefillChunk:
    m = model_tensors()
    if m.prefill_full is not None:
        raise RuntimeError("the exported prefill runs the whole prompt as one chunk: bind_prefill_tensors(prompt_ids, "
                           "chunk=len(prompt_ids))")
    return _chunk("tail")


def run_embed_tokens(rt: RuntimeSession) -> None:
    """Every prompt token's embedding row (src/models/quantized_qwen3/dispatch/embed_tokens.py:11-16)."""
    _run_embed_tokens_with_tensors(rt, _whole_prompt().embed)


def run_text_layer(rt: RuntimeSession, layer_idx: int, *, rope_theta: float = 1.0e6) -> None:
    """One decoder layer over the whole prompt at positions 0.. with causal attention
    (src/models/quantized_qwen3/dispatch/text_layer.py:33-106); the first layer also fills the prompt's RoPE
    table and mask tiles."""
    ch = _whole_prompt()
    if layer_idx == 0:
        V.ROPE_TABLE_F32(rt, start_position=ch.start, theta=rope_theta, cos=ch.rope.cos, sin=ch.rope.sin)
        V.FA_MASK_OPT_F16(rt, mask=ch.causal_mask, output=ch.mask_opt)
    _run_text_layer_with_tensors(rt, ch.layers[layer_idx], ch)


def run_text_norm_all(rt: RuntimeSession, output: torch.Tensor) -> None:
    """The exported run_text_norm (src/models/quantized_qwen3/dispatch/text_norm.py:11-16): the final RMSNorm of
    every prompt position, fp32 or bf16 [1, T, H] into ``output``."""
    ch = _whole_prompt()
    m = model_tensors()
    V.RMS_NORM_MUL_F32(rt, x=ch.embed.embedding, weight=m.text_norm.p_weight, output=output)
