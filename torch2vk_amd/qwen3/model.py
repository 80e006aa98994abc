"""Qwen3 greedy decode on MI355X: the reference's decode-step surface over libt2h.

One decode step (src/models/optimized_qwen3/run.py:142-172) is, per token:

    embed                                   1 launch   (EMBEDDING_Q4_K_F32)
    per layer                               5 launches (6 with a Q6_K v_proj):
      RMSNorm + Q|K|V GEMV                  (RMS_NORM_MUL + LINEAR_NOBIAS_Q4_K_QKV_MATVEC, or
                                             LINEAR_NOBIAS_Q4_QK_Q6_V_MATVEC as Q4_K q|k + Q6_K v)
      q/k-norm + RoPE + KV write + attention (RMS_NORM_ROPE_TRANSPOSE x2 + SDPA_DECODE_CACHE_WRITE;
                                             a split-K pass and a merge pass)
      o_proj GEMV + residual                (LINEAR_NOBIAS_Q4_K_MATVEC_ADD / _Q6_K_)
      RMSNorm + gate|up GEMV + SwiGLU       (RMS_NORM_MUL + LINEAR_NOBIAS_Q4_K_QK_MATVEC + SWIGLU)
      down GEMV + residual                  (LINEAR_NOBIAS_Q4_K_MATVEC_ADD / _Q6_K_)
    final RMSNorm + LM head + argmax        1 launch   (run_decode_norm + LM_HEAD_{Q4_K,Q6_K}_ARGMAX_PARTIAL)
    token select + store + advance          1 launch   (QWEN3_TOKEN_SELECT_REDUCE_* + QWEN3_TOKEN_STORE_EOS)

Weights are Q4_K (uniform int4) or follow the Q4_K_M policy (Q6_K for v/down
on the more-bits layers and for the LM head); each linear runs the GEMV of
its own type.

The reference runs 10 dispatches per layer and waits on the host every token
(src/torch2vk/runtime/replay.py:260-261).  Here every dynamic scalar (cache
position, token index, the token itself) lives in device memory, so whole
steps are captured into one HIP graph and replayed with no host round trip.

The residual stream is fp32; GEMV inputs are bf16; the KV cache is bf16
token-major [S, NK, D] per layer (the reference's optimized cache layout,
src/models/optimized_qwen3/tensors/model.py:104-150, in bf16 instead of fp16).
"""

from __future__ import annotations

import torch

from torch2vk_amd import kernels
from torch2vk_amd.qwen3.config import Qwen3Config
from torch2vk_amd.qwen3.weights import Qwen3Weights

LM_HEAD_PARTIALS = 512


def _check_types(c: Qwen3Config, types: dict[str, str]) -> None:
    """The decode path runs Q4_K everywhere and Q6_K where the Q4_K_M policy puts it (v, down,
    lm_head); anything else has no decode kernel here and is refused up front."""
    allowed = {"embed": ("q4_k", "q8_0"), "lm_head": ("q4_k", "q6_k")}
    for i in range(c.layers):
        for n in ("q", "k", "gate", "up"):
            allowed[f"layers.{i}.{n}"] = ("q4_k",)
        for n in ("v", "o", "down"):
            allowed[f"layers.{i}.{n}"] = ("q4_k", "q6_k")
    for name, t in types.items():
        if name in allowed and t not in allowed[name]:
            raise NotImplementedError(f"{name}: no {t} decode kernel (built: {allowed[name]})")


class Qwen3Decoder:
    """Greedy decoder over libt2h.  ``persistent`` selects how a token's layers run: one persistent launch
    for all of them (t2h_qwen3_decode_layers: the 8B and 0.6B shapes with Q4_K weights, v and down Q4_K or
    Q6_K as the uniform and Q4_K_M policies give them), or one launch per op (run_decode_layer, every shape and
    weight mix).  None (the default) picks the persistent kernel when it
    applies: on MI355X it saves the launch and ramp of ~250 kernels per token."""

    PREFILL_GRAPHS = 4  # captured prefill graphs kept (prefill_graphed)

    def __init__(self, weights: Qwen3Weights, *, max_positions: int, max_new_tokens: int, device=None,
                 persistent: bool | None = None,
                 kv_cache: tuple[torch.Tensor, torch.Tensor] | None = None) -> None:
        c = weights.config
        self.config: Qwen3Config = c
        self.weights = weights
        self.types = dict(weights.types)
        _check_types(c, self.types)
        dev = torch.device(device) if device is not None else weights.packed["embed"].device
        self.device = dev
        self.max_positions = max_positions
        bf, f32 = torch.bfloat16, torch.float32
        if kv_cache is None:
            self.k_cache = torch.zeros(c.layers, max_positions, c.kv_heads, c.head_dim, dtype=bf, device=dev)
            self.v_cache = torch.zeros_like(self.k_cache)
        else:
            # caller-owned bf16 [layers, max_positions, kv_heads, head_dim] views, each layer's rows contiguous
            # (a Qwen3DecoderGroup's layer-major caches)
            want = (c.layers, max_positions, c.kv_heads, c.head_dim)
            for t in kv_cache:
                if (tuple(t.shape) != want or t.dtype != bf or t.device != dev or not t[0].is_contiguous()
                        or t.stride(1) != c.kv_heads * c.head_dim):
                    raise ValueError(f"kv_cache tensors must be bf16 {want} on {dev} with contiguous layers")
            self.k_cache, self.v_cache = kv_cache
        self.h = torch.zeros(c.hidden, dtype=f32, device=dev)
        self.q = torch.zeros(c.q_dim, dtype=f32, device=dev)
        self.k = torch.zeros(c.kv_dim, dtype=f32, device=dev)
        self.v = torch.zeros(c.kv_dim, dtype=f32, device=dev)
        self.attn = torch.zeros(c.q_dim, dtype=bf, device=dev)
        self.act = torch.zeros(c.mlp, dtype=bf, device=dev)
        self.attn_ws = kernels.attn_decode_workspace(c.heads, c.kv_heads, c.head_dim, max_positions, dev)
        self.partial_scores = torch.zeros(LM_HEAD_PARTIALS, dtype=f32, device=dev)
        self.partial_tokens = torch.zeros(LM_HEAD_PARTIALS, dtype=torch.int32, device=dev)
        self.next_token = torch.zeros(1, 1, dtype=torch.int64, device=dev)
        self.done = torch.zeros(1, dtype=torch.int32, device=dev)
        self.generated = torch.full((max_new_tokens,), -1, dtype=torch.int64, device=dev)
        self.length = torch.zeros(1, dtype=torch.int32, device=dev)
        self.stopped = torch.zeros(1, dtype=torch.int32, device=dev)
        self.position = torch.zeros(1, dtype=torch.int32, device=dev)
        self.eos = torch.tensor(c.eos_token_ids, dtype=torch.int64, device=dev)
        self.stop_on_eos = True
        self._graphs: dict[int, torch.cuda.CUDAGraph] = {}
        self._prefill_graphs: dict[tuple[int, int, int, bool], tuple[torch.cuda.CUDAGraph, torch.Tensor]] = {}
        self.persistent = False
        self.status = torch.zeros(1, dtype=torch.int32, device=dev)
        if persistent is not False:
            why = self._persistent_unsupported()
            if why is None:
                self.layers_ws = kernels.decode_layers_workspace(c.hidden, c.mlp, c.heads, c.kv_heads, c.head_dim, dev)
                self.layer_table = kernels.decode_layer_table(weights.packed, weights.norms, c.layers, self.k_cache,
                                                              self.v_cache, self.types)
                self.persistent = True
            elif persistent:
                raise NotImplementedError(f"persistent decode kernel: {why}")

    def _persistent_unsupported(self) -> str | None:
        c = self.config
        if not kernels.decode_layers_supported(c.hidden, c.mlp, c.heads, c.kv_heads, c.head_dim):
            return f"shape hidden={c.hidden} mlp={c.mlp} heads={c.heads}/{c.kv_heads} d={c.head_dim} not built"
        if self.max_positions > 8192:
            return "KV capacity above 8192 positions"
        if self.config.layers > 64:
            return "more than 64 layers"
        for i in range(c.layers):
            t = {n: self.types[f"layers.{i}.{n}"] for n in ("q", "k", "v", "o", "gate", "up", "down")}
            if any(t[n] != "q4_k" for n in ("q", "k", "o", "gate", "up")):
                return "q, k, o, gate or up weights other than Q4_K"
            if any(t[n] not in ("q4_k", "q6_k") for n in ("v", "down")):
                return "v or down weights other than Q4_K or Q6_K"
            q, k, v = (self.weights.packed[f"layers.{i}.{n}"] for n in ("q", "k", "v"))
            if k.data_ptr() != q.data_ptr() + q.numel():
                return "q and k rows are not stacked in one allocation"
            if t["v"] == "q4_k" and v.data_ptr() != k.data_ptr() + k.numel():
                return "a Q4_K v does not follow k's rows in the same allocation"
        return None

    def check_status(self) -> None:
        """Raise if a grid barrier of the persistent kernel ever timed out (its results are then invalid)."""
        if not self.persistent:
            return
        code = int(self.status.item())
        if code != 0:
            phases = {1: "qkv", 2: "attention q", 3: "attention k/v", 4: "merge", 5: "o", 6: "gate/up", 7: "down"}
            where = f"layer {(code >> 8) & 0xff}, phase {phases.get(code & 0xff, code & 0xff)}"
            raise RuntimeError(f"persistent decode kernel: a wait for another block timed out at {where} "
                               f"(status {code:#x}); results are invalid")

    # ----------------------------------------------------------- state --

    def reset(self, position: int = 0, token: int | None = None) -> None:
        self.position.fill_(position)
        self.length.zero_()
        self.stopped.zero_()
        self.done.zero_()
        self.generated.fill_(-1)
        if token is not None:
            self.next_token.fill_(token)

    def _w(self, name: str) -> torch.Tensor:
        return self.weights.packed[name]

    def _n(self, name: str) -> torch.Tensor:
        return self.weights.norms[name]

    # ------------------------------------------- reference op surface --

    def run_decode_embed(self) -> None:
        """Token -> fp32 residual stream (run_decode_embed, EMBEDDING_Q4_K_F32 / EMBEDDING_Q8_0_F32)."""
        self.embed_tokens(self.next_token.view(-1), out=self.h.view(1, -1))

    def embed_tokens(self, ids: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
        """fp32 [len(ids), hidden] rows of the token embedding (run_embed_tokens)."""
        fn = kernels.embedding_q8_0 if self.types["embed"] == "q8_0" else kernels.embedding_q4_k
        return fn(self._w("embed"), ids, self.config.hidden, out=out)

    def run_decode_layer(self, layer_idx: int, *, cache_position: int | None = None) -> None:
        """One decoder layer at the device-resident position
        (run_decode_layer, src/models/optimized_qwen3/dispatch/decode_layer.py:131-136).
        A Python ``cache_position`` is written to the device counter first."""
        if cache_position is not None:
            self.position.fill_(cache_position)
        p = f"layers.{layer_idx}."
        self._qkv(layer_idx)
        self._attention(layer_idx)
        self._linear_residual(self.attn, p + "o")
        self._gate_up(layer_idx)
        self._linear_residual(self.act, p + "down")

    def _qkv(self, layer_idx: int) -> None:
        """RMSNorm + Q|K|V.  The Q4_K parts share one launch; a Q6_K v (Q4_K_M more-bits layers) runs
        its own RMSNorm-prologue GEMV (the reference fuses it as LINEAR_NOBIAS_Q4_QK_Q6_V_MATVEC_F32)."""
        c, t, p = self.config, self.types, f"layers.{layer_idx}."
        q4 = [(n, o) for n, o in (("q", self.q), ("k", self.k), ("v", self.v)) if t[p + n] == "q4_k"]
        kernels.q4k_matvec_multi(self.h, [self._w(p + n) for n, _ in q4], [o for _, o in q4],
                                 norm_weight=self._n(p + "input_norm"), eps=c.rms_eps)
        if t[p + "v"] == "q6_k":
            kernels.qx_matvec(self.h, self._w(p + "v"), "q6_k", out=self.v, norm_weight=self._n(p + "input_norm"),
                              eps=c.rms_eps)

    def _attention(self, layer_idx: int) -> None:
        c, p = self.config, f"layers.{layer_idx}."
        kernels.attn_decode(self.q, self.k, self.v, self.k_cache[layer_idx], self.v_cache[layer_idx], self.attn,
                            self.position, self.attn_ws, q_norm_weight=self._n(p + "q_norm"),
                            k_norm_weight=self._n(p + "k_norm"), theta=c.rope_theta, eps=c.rms_eps)

    def _gate_up(self, layer_idx: int) -> None:
        p = f"layers.{layer_idx}."
        kernels.q4k_rmsnorm_swiglu(self.h, self._n(p + "post_norm"), self._w(p + "gate"), self._w(p + "up"),
                                   self.act, eps=self.config.rms_eps)

    def _linear_residual(self, x: torch.Tensor, name: str) -> None:
        """h += x . deq(W)^T with the kernel of W's type (_linear_q4_or_q6,
        src/models/optimized_qwen3/dispatch/decode_layer.py:22-58; one row, so a GEMV)."""
        kernels.quantized_linear(x, self._w(name), self.types[name], out=self.h, residual=self.h)

    def _lm_head(self) -> None:
        if self.types["lm_head"] == "q4_k" and self.config.hidden in (1024, 4096):
            # the multi-sequence head kernel with one sequence: the same partials, 10-20 % faster
            kernels.q4k_lm_head_argmax_partial_seqs([self.h], self._w("lm_head"), [self.partial_scores],
                                                    [self.partial_tokens], norm_weight=self._n("norm"),
                                                    eps=self.config.rms_eps)
            return
        kernels.lm_head_argmax_partial(self.h, self._w("lm_head"), self.types["lm_head"], self.partial_scores,
                                       self.partial_tokens, norm_weight=self._n("norm"), eps=self.config.rms_eps)

    def run_lm_head_select(self) -> None:
        """Final RMSNorm + LM head + argmax + EOS flag (run_decode_norm + _run_lm_head_select,
        src/models/optimized_qwen3/run.py:116-139); logits are never materialised."""
        self._lm_head()
        kernels.token_select(self.partial_scores, self.partial_tokens, self.eos, self.next_token, self.done)

    def run_token_store(self, advance: bool = True) -> None:
        """QWEN3_TOKEN_STORE_EOS_F32 with the token index read from the device length counter."""
        kernels.token_store(self.next_token, self.done, self.generated, self.length, self.stopped,
                            stop_on_eos=self.stop_on_eos, token_index_ptr=self.length,
                            advance=self.position if advance else None)

    def logits(self, h: torch.Tensor | None = None) -> torch.Tensor:
        """fp32 [vocab] logits of one residual-stream row (default: the decoder's own h): final RMSNorm -> bf16 ->
        LM-head GEMV of the head's type.  A decode step's fused LM head + argmax never writes these; they are
        for checking a step's token against its scores."""
        c = self.config
        h = self.h if h is None else h
        x = kernels.rms_norm(h.reshape(1, c.hidden), self._n("norm"),
                             out=torch.empty(1, c.hidden, dtype=torch.bfloat16, device=self.device), eps=c.rms_eps)
        return kernels.quantized_linear(x, self._w("lm_head"), self.types["lm_head"]).view(-1)

    def step_logits(self, position: int, *, token: int | None = None,
                    embed: torch.Tensor | None = None) -> torch.Tensor:
        """fp32 [vocab] logits of the decode step at ``position`` over the cache rows 0..position-1 as they stand,
        its input the embedding of ``token`` or the fp32 row ``embed``: the same layer launches as a decode step,
        then ``logits``.  The decoder's position, token, residual stream and the cache rows at ``position`` are
        restored afterwards, so a finished generation can be re-examined step by step."""
        if (token is None) == (embed is None):
            raise ValueError("pass token or embed")
        if not 0 <= position < self.max_positions:
            raise ValueError(f"position {position} outside the KV capacity {self.max_positions}")
        saved = [t.clone() for t in (self.position, self.next_token, self.h, self.k_cache[:, position],
                                     self.v_cache[:, position])]
        self.position.fill_(position)
        if embed is None:
            self.next_token.fill_(int(token))
            self.run_decode_embed()
        else:
            self.h.copy_(embed.reshape(-1))
        self.run_decode_layers()
        out = self.logits()
        self.check_status()
        for dst, src in zip((self.position, self.next_token, self.h, self.k_cache[:, position],
                             self.v_cache[:, position]), saved):
            dst.copy_(src)
        return out

    def run_decode_layers(self, trace: torch.Tensor | None = None) -> None:
        """Every layer at the device-resident position: one persistent launch, or one launch per op.
        ``trace`` (kernels.decode_layers_trace) records the persistent launch's phase timeline."""
        if self.persistent:
            c = self.config
            kernels.decode_layers(self.layer_table, self.h, self.position, self.layers_ws, self.status,
                                  hidden=c.hidden, mlp=c.mlp, nh=c.heads, nk=c.kv_heads, d=c.head_dim,
                                  s_cap=self.max_positions, eps=c.rms_eps, theta=c.rope_theta, trace=trace)
        else:
            for i in range(self.config.layers):
                self.run_decode_layer(i)

    def forward_token(self) -> None:
        """Embed next_token at the current position, run every layer, select the next token."""
        self.run_decode_embed()
        self.run_decode_layers()
        self.run_lm_head_select()

    def decode_step(self) -> None:
        """One full greedy step: forward, select + store the token, advance the position."""
        self.run_decode_embed()
        self.run_decode_layers()
        self.run_step_tail()

    def run_step_tail(self) -> None:
        """The end of a decode step after the layers: LM head, select + store the token, advance the position."""
        self._lm_head()
        self._select_store()

    def _select_store(self) -> None:
        """Reduce the LM head's partials to the greedy token, store it, advance the position."""
        kernels.token_select_store(self.partial_scores, self.partial_tokens, self.eos, self.next_token, self.done,
                                   self.generated, self.length, self.stopped, stop_on_eos=self.stop_on_eos,
                                   advance=self.position)

    # ------------------------------------------------------ HIP graphs --

    def graph(self, steps: int) -> torch.cuda.CUDAGraph:
        """A graph of ``steps`` consecutive decode steps (captured once per step count)."""
        if steps not in self._graphs:
            saved = self._save_state()
            side = torch.cuda.Stream(device=self.device)
            side.wait_stream(torch.cuda.current_stream(self.device))
            with torch.cuda.stream(side):
                self.decode_step()  # warm-up launch outside capture
            torch.cuda.current_stream(self.device).wait_stream(side)
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                for _ in range(steps):
                    self.decode_step()
            self._restore_state(saved)
            self._graphs[steps] = g
        return self._graphs[steps]

    def _save_state(self):
        return [t.clone() for t in (self.position, self.length, self.stopped, self.done, self.next_token,
                                    self.generated)]

    def _restore_state(self, saved) -> None:
        for dst, src in zip((self.position, self.length, self.stopped, self.done, self.next_token, self.generated),
                            saved):
            dst.copy_(src)

    def run_steps(self, n: int, steps_per_graph: int = 8, use_graph: bool = True) -> None:
        if not use_graph:
            for _ in range(n):
                self.decode_step()
            return
        full, rest = divmod(n, steps_per_graph)
        if full:
            g = self.graph(steps_per_graph)
            for _ in range(full):
                g.replay()
        for _ in range(rest):
            self.decode_step()

    # ------------------------------------------------------- generate --

    def prefill(self, prompt_ids: torch.Tensor, start: int = 0) -> None:
        """Feed the prompt one token at a time (KV cache fill); the last prompt token's step stores the
        first generated token."""
        ids = prompt_ids.to(device=self.device, dtype=torch.int64).view(-1)
        self.reset(position=start)
        for i in range(ids.numel()):
            self.next_token.view(-1).copy_(ids[i:i + 1])
            self.forward_token()
            if i + 1 < ids.numel():
                self.position.add_(1)
        self.run_token_store(advance=True)

    # ------------------------------------------------- chunked prefill --

    def _fused_qkv(self, layer_idx: int) -> torch.Tensor | None:
        """The layer's q|k|v rows as one matrix when they are stacked in one allocation of one type."""
        p = f"layers.{layer_idx}."
        q, k, v = (self._w(p + n) for n in ("q", "k", "v"))
        if len({self.types[p + n] for n in ("q", "k", "v")}) != 1:
            return None
        if k.data_ptr() != q.data_ptr() + q.numel() or v.data_ptr() != k.data_ptr() + k.numel():
            return None
        rows = q.shape[0] + k.shape[0] + v.shape[0]
        return q.as_strided((rows, q.shape[1]), (q.shape[1], 1))

    def _prefill_layer(self, i: int, h: torch.Tensor, start: int, mask: torch.Tensor | None = None,
                       mask_tiles: torch.Tensor | None = None) -> None:
        """One layer over a chunk's fp32 residual stream h [n, hidden] at positions start.. (run_text_layer,
        src/models/optimized_qwen3/dispatch/text_layer.py): RMSNorm rows -> q|k|v GEMM -> q/k norm + RoPE +
        KV cache write -> causal flash attention over the cache -> o GEMM + residual -> RMSNorm -> gate|up
        GEMM with SwiGLU in its epilogue -> down GEMM + residual.  GEMMs run on the matrix cores for any chunk length.
        ``mask`` (additive fp32 [1, n, start + n]) replaces causality in the attention; ``mask_tiles`` are its
        tile classes (kernels.fa_mask_tiles), computed once for every layer of a pass."""
        c, t, p = self.config, self.types, f"layers.{i}."
        n = h.shape[0]
        x = kernels.rms_norm(h, self._n(p + "input_norm"), out=torch.empty(n, c.hidden, dtype=torch.bfloat16,
                                                                           device=self.device), eps=c.rms_eps)
        fused = self._fused_qkv(i)
        if fused is not None:
            qkv = kernels.quantized_linear(x, fused, t[p + "q"], out_dtype=torch.float32)
            q, k, v = qkv[:, :c.q_dim], qkv[:, c.q_dim:c.q_dim + c.kv_dim], qkv[:, c.q_dim + c.kv_dim:]
        else:
            q, k, v = (kernels.quantized_linear(x, self._w(p + nm), t[p + nm], out_dtype=torch.float32)
                       for nm in ("q", "k", "v"))
        qb = torch.empty(n, c.heads, c.head_dim, dtype=torch.bfloat16, device=self.device)
        kernels.qk_norm_rope_cache(q, k, v, qb, self.k_cache[i], self.v_cache[i], start,
                                   q_norm_weight=self._n(p + "q_norm"), k_norm_weight=self._n(p + "k_norm"),
                                   theta=c.rope_theta, eps=c.rms_eps)
        keys = self.k_cache[i, :start + n].unsqueeze(0)
        vals = self.v_cache[i, :start + n].unsqueeze(0)
        if mask is None:
            attn = kernels.flash_attn_prefill(qb.unsqueeze(0), keys, vals, causal=True, causal_offset=start)
        else:
            attn = kernels.flash_attn_prefill(qb.unsqueeze(0), keys, vals, causal=False, mask=mask,
                                              mask_tiles=mask_tiles)
        kernels.quantized_linear(attn.view(n, c.q_dim), self._w(p + "o"), t[p + "o"], out=h, residual=h)
        x = kernels.rms_norm(h, self._n(p + "post_norm"), out=x, eps=c.rms_eps)
        if t[p + "gate"] == t[p + "up"] and n > kernels.GEMV_MAX_ROWS:
            act = kernels.gemm_swiglu(x, self._w(p + "gate"), self._w(p + "up"), t[p + "gate"])
        else:
            gate = kernels.quantized_linear(x, self._w(p + "gate"), t[p + "gate"], out_dtype=torch.float32)
            up = kernels.quantized_linear(x, self._w(p + "up"), t[p + "up"], out_dtype=torch.float32)
            act = kernels.swiglu(gate, up)
            del gate, up
        kernels.quantized_linear(act, self._w(p + "down"), t[p + "down"], out=h, residual=h)

    def forward_masked(self, embeds: torch.Tensor, mask: torch.Tensor) -> torch.Tensor:
        """OmniVoice's LLM pass (src/models/quantized_omnivoice/dispatch/llm_forward.py:19-70): every layer over
        the whole sequence of input embeddings [T, hidden] at positions 0..T-1, attention under the additive
        mask [T, T] (SDPA_MASKED_F32; -inf where a key is hidden) instead of causality, then the final RMSNorm
        of every position -> fp32 [T, hidden].  The layers' K/V go to rows 0..T-1 of the KV cache.  The same
        kernels as the chunked prefill: matrix-core GEMMs of each weight's type and masked flash attention."""
        c = self.config
        e = embeds.to(device=self.device, dtype=torch.float32).reshape(-1, c.hidden)
        t_len = e.shape[0]
        if t_len > self.max_positions:
            raise ValueError(f"{t_len} positions exceed the KV capacity {self.max_positions}")
        m = mask.to(device=self.device, dtype=torch.float32).reshape(1, t_len, t_len).contiguous()
        h = e.clone()
        tiles = kernels.fa_mask_tiles(m)  # FA_MASK_OPT_F16 once per pass (src/models/optimized_qwen3/run.py:406)
        for i in range(c.layers):
            self._prefill_layer(i, h, 0, mask=m, mask_tiles=tiles)
        return kernels.rms_norm(h, self._n("norm"), out=torch.empty_like(h), eps=c.rms_eps)

    def prefill_chunked(self, prompt_ids: torch.Tensor | None = None, *, embeds: torch.Tensor | None = None,
                        start: int = 0, chunk: int = 2048) -> None:
        """Prompt (token ids, or fp32 input embeddings [T, hidden]) through the matrix-core path ``chunk``
        tokens at a time -- the reference's fixed-size chunk + tail prefill (src/models/optimized_qwen3/
        run.py:395-471) with every chunk a plain GEMM pass and causal attention that visits only the key tiles
        at or below each query tile's diagonal.  Then the last token's final norm, LM head and greedy select,
        and the first generated token stored, as after ``prefill``."""
        c = self.config
        if (prompt_ids is None) == (embeds is None):
            raise ValueError("pass prompt_ids or embeds")
        if embeds is None:
            ids = prompt_ids.to(device=self.device, dtype=torch.int64).view(-1)
            e = self.embed_tokens(ids)
        else:
            e = embeds.reshape(-1, c.hidden)
            if e.dtype != torch.float32 or e.device != self.device:
                raise ValueError("embeds must be fp32 on the decoder's device")
        total = e.shape[0]
        if total == 0:
            raise ValueError("empty prompt")
        if start + total > self.max_positions:
            raise ValueError("prompt exceeds the KV cache capacity")
        if chunk <= 0:
            raise ValueError("chunk must be positive")
        self.reset(position=start)
        for c0 in range(0, total, chunk):
            h = e[c0:c0 + chunk].clone()
            for i in range(c.layers):
                self._prefill_layer(i, h, start + c0)
        self.h.copy_(h[-1])
        self.position.fill_(start + total - 1)
        self.run_lm_head_select()
        self.run_token_store(advance=True)

    def prefill_graphed(self, prompt_ids: torch.Tensor, *, start: int = 0, chunk: int = 2048) -> None:
        """prefill_chunked of a token-id prompt replayed from a HIP graph: the first call for a (length, start,
        chunk, stop_on_eos) captures the whole prefill (every layer's launches, the LM head and the token store)
        reading the ids from a buffer of the decoder's; later calls copy the ids into that buffer and replay.
        Results are prefill_chunked's bit for bit; a short prompt's prefill is bound by launch overhead, which the
        graph removes.  Each captured graph keeps a memory pool holding every intermediate of one whole prefill
        (about the GEMM activations of one chunk), so at most PREFILL_GRAPHS of them are kept, least recently
        used first out; ``clear_prefill_graphs`` drops them all."""
        ids = prompt_ids.to(device=self.device, dtype=torch.int64).view(-1)
        if ids.numel() == 0:
            raise ValueError("empty prompt")
        # stop_on_eos is read on the host when the token store is launched, so the capture freezes it
        key = (ids.numel(), start, chunk, bool(self.stop_on_eos))
        if key in self._prefill_graphs:
            self._prefill_graphs[key] = self._prefill_graphs.pop(key)  # most recently used last
        else:
            while len(self._prefill_graphs) >= self.PREFILL_GRAPHS:
                self._prefill_graphs.pop(next(iter(self._prefill_graphs)))
            buf = ids.clone()
            side = torch.cuda.Stream(device=self.device)
            side.wait_stream(torch.cuda.current_stream(self.device))
            with torch.cuda.stream(side):
                self.prefill_chunked(buf, start=start, chunk=chunk)  # warm-up launch outside capture
            torch.cuda.current_stream(self.device).wait_stream(side)
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                self.prefill_chunked(buf, start=start, chunk=chunk)
            self._prefill_graphs[key] = (g, buf)
        g, buf = self._prefill_graphs[key]
        buf.copy_(ids)
        g.replay()

    def clear_prefill_graphs(self) -> None:
        """Drop every captured prefill graph and its memory pool."""
        self._prefill_graphs.clear()

    def prefill_embeds(self, embeds: torch.Tensor, start: int = 0) -> None:
        """Feed a prompt given as fp32 input embeddings [T, hidden] -- a Qwen3-ASR prompt after the audio
        features were injected (run_audio_inject) -- one position at a time; the last position's step selects
        and stores the first generated token."""
        c = self.config
        e = embeds.reshape(-1, c.hidden)
        if e.dtype != torch.float32 or e.device != self.device:
            raise ValueError("embeds must be fp32 on the decoder's device")
        if e.shape[0] == 0:
            raise ValueError("empty prompt")
        self.reset(position=start)
        for i in range(e.shape[0]):
            self.h.copy_(e[i])
            self.run_decode_layers()
            if i + 1 < e.shape[0]:
                self.position.add_(1)
        self.run_lm_head_select()
        self.run_token_store(advance=True)

    def _check_budget(self, prompt_len: int, max_new_tokens: int) -> None:
        if max_new_tokens > self.generated.numel():
            raise ValueError("max_new_tokens exceeds the decoder's generated-token buffer")
        if prompt_len + max_new_tokens > self.max_positions:
            raise ValueError("prompt + new tokens exceed the KV cache capacity")

    def _finish(self, max_new_tokens: int, steps_per_graph: int, use_graph: bool) -> list[int]:
        self.run_steps(max_new_tokens - 1, steps_per_graph=steps_per_graph, use_graph=use_graph)
        n = int(self.length.item())
        self.check_status()
        return self.generated[:n].tolist()

    def generate(self, prompt_ids: torch.Tensor, max_new_tokens: int, *, steps_per_graph: int = 8,
                 use_graph: bool = True, prefill_chunk: int | None = None) -> list[int]:
        """Greedy decode.  ``prefill_chunk`` set: the prompt goes through the chunked matrix-core prefill;
        None: one decode step per prompt token."""
        self._check_budget(prompt_ids.numel(), max_new_tokens)
        if prefill_chunk:
            self.prefill_chunked(prompt_ids, chunk=prefill_chunk)
        else:
            self.prefill(prompt_ids)
        return self._finish(max_new_tokens, steps_per_graph, use_graph)

    def generate_from_embeds(self, embeds: torch.Tensor, max_new_tokens: int, *, steps_per_graph: int = 8,
                             use_graph: bool = True, prefill_chunk: int | None = None) -> list[int]:
        """Greedy decode after a prompt of input embeddings (the Qwen3-ASR transcription loop)."""
        self._check_budget(embeds.reshape(-1, self.config.hidden).shape[0], max_new_tokens)
        if prefill_chunk:
            self.prefill_chunked(embeds=embeds, chunk=prefill_chunk)
        else:
            self.prefill_embeds(embeds)
        return self._finish(max_new_tokens, steps_per_graph, use_graph)


class Qwen3DecoderGroup:
    """Several persistent decoders (each with its own KV cache, position and tokens; typically one set of
    weights) stepped together: one persistent launch runs every sequence's layers
    (t2h_qwen3_decode_layers_seqs), then each sequence's embedding, LM head and token store run as usual.
    Built for 4 sequences of the Qwen3-0.6B shape, as in the Qwen3-ASR job's utterances.  A group made by
    ``create`` keeps its sequences' caches layer-major ([layers, n_seq, positions, kv heads, dim]), so equal-
    length prompts can also be prefilled as one batch (``prefill_chunked``)."""

    @classmethod
    def create(cls, weights: Qwen3Weights, n_seq: int, *, max_positions: int, max_new_tokens: int,
               device=None) -> "Qwen3DecoderGroup":
        c = weights.config
        dev = torch.device(device) if device is not None else weights.packed["embed"].device
        shape = (c.layers, n_seq, max_positions, c.kv_heads, c.head_dim)
        k = torch.zeros(shape, dtype=torch.bfloat16, device=dev)
        v = torch.zeros_like(k)
        decs = [Qwen3Decoder(weights, max_positions=max_positions, max_new_tokens=max_new_tokens, device=dev,
                             persistent=True, kv_cache=(k[:, b], v[:, b])) for b in range(n_seq)]
        group = cls(decs)
        group.k_cache, group.v_cache = k, v
        return group

    def __init__(self, decoders: list[Qwen3Decoder]) -> None:
        if len(decoders) not in kernels.DECODE_SEQS:
            raise ValueError(f"a group runs {kernels.DECODE_SEQS} sequences, got {len(decoders)}")
        d0 = decoders[0]
        for d in decoders:
            if not d.persistent:
                raise ValueError("every decoder of a group must run the persistent kernel")
            if d.config != d0.config or d.max_positions != d0.max_positions or d.device != d0.device:
                raise ValueError("a group's decoders must share the shape, KV capacity and device")
        self.decoders = decoders
        self._graphs: dict[int, torch.cuda.CUDAGraph] = {}
        self.k_cache: torch.Tensor | None = None  # layer-major caches of a group made by create()
        self.v_cache: torch.Tensor | None = None

    def _prefill_layer(self, i: int, h: torch.Tensor, n_seq: int, start: int) -> None:
        """Qwen3Decoder._prefill_layer for n_seq sequences of n tokens each (h [n_seq n, hidden], sequence-major
        rows) at positions start..: the GEMMs and norms over all rows at once, the q/k prologue into every
        sequence's cache in one launch, and causal flash attention over the batch of caches."""
        d0 = self.decoders[0]
        c, t, p = d0.config, d0.types, f"layers.{i}."
        rows = h.shape[0]
        n = rows // n_seq
        x = kernels.rms_norm(h, d0._n(p + "input_norm"),
                             out=torch.empty(rows, c.hidden, dtype=torch.bfloat16, device=d0.device), eps=c.rms_eps)
        fused = d0._fused_qkv(i)
        if fused is not None:
            qkv = kernels.quantized_linear(x, fused, t[p + "q"], out_dtype=torch.float32)
            q, k, v = qkv[:, :c.q_dim], qkv[:, c.q_dim:c.q_dim + c.kv_dim], qkv[:, c.q_dim + c.kv_dim:]
        else:
            q, k, v = (kernels.quantized_linear(x, d0._w(p + nm), t[p + nm], out_dtype=torch.float32)
                       for nm in ("q", "k", "v"))
        qb = torch.empty(rows, c.heads, c.head_dim, dtype=torch.bfloat16, device=d0.device)
        kernels.qk_norm_rope_cache(q, k, v, qb, self.k_cache[i], self.v_cache[i], start,
                                   q_norm_weight=d0._n(p + "q_norm"), k_norm_weight=d0._n(p + "k_norm"),
                                   theta=c.rope_theta, eps=c.rms_eps)
        keys = self.k_cache[i, :, :start + n]
        vals = self.v_cache[i, :, :start + n]
        attn = kernels.flash_attn_prefill(qb.view(n_seq, n, c.heads, c.head_dim), keys, vals, causal=True,
                                          causal_offset=start)
        kernels.quantized_linear(attn.view(rows, c.q_dim), d0._w(p + "o"), t[p + "o"], out=h, residual=h)
        x = kernels.rms_norm(h, d0._n(p + "post_norm"), out=x, eps=c.rms_eps)
        if t[p + "gate"] == t[p + "up"] and rows > kernels.GEMV_MAX_ROWS:
            act = kernels.gemm_swiglu(x, d0._w(p + "gate"), d0._w(p + "up"), t[p + "gate"])
        else:
            gate = kernels.quantized_linear(x, d0._w(p + "gate"), t[p + "gate"], out_dtype=torch.float32)
            up = kernels.quantized_linear(x, d0._w(p + "up"), t[p + "up"], out_dtype=torch.float32)
            act = kernels.swiglu(gate, up)
            del gate, up
        kernels.quantized_linear(act, d0._w(p + "down"), t[p + "down"], out=h, residual=h)

    def prefill_chunked(self, embeds: list[torch.Tensor], *, start: int = 0, chunk: int = 2048) -> None:
        """Every sequence's prompt of input embeddings (fp32 [T, hidden], the same T for all) through the
        matrix-core prefill as one batch, ``chunk`` positions at a time; then, per sequence, the last token's
        final norm, LM head and greedy select, and the first generated token stored (as
        Qwen3Decoder.prefill_chunked, which a group of one equals)."""
        if self.k_cache is None:
            raise ValueError("batched prefill needs a group made by Qwen3DecoderGroup.create")
        ds, c = self.decoders, self.decoders[0].config
        if len(embeds) != len(ds):
            raise ValueError(f"one prompt per sequence: {len(ds)}, got {len(embeds)}")
        e = [x.reshape(-1, c.hidden) for x in embeds]
        total = e[0].shape[0]
        if total == 0 or any(x.shape[0] != total for x in e):
            raise ValueError("the prompts must be non-empty and of one length")
        if any(x.dtype != torch.float32 or x.device != ds[0].device for x in e):
            raise ValueError("embeds must be fp32 on the decoders' device")
        if start + total > ds[0].max_positions:
            raise ValueError("prompt exceeds the KV cache capacity")
        if chunk <= 0:
            raise ValueError("chunk must be positive")
        n_seq = len(ds)
        stacked = torch.stack(e)  # [n_seq, T, hidden]
        for d in ds:
            d.reset(position=start)
        for c0 in range(0, total, chunk):
            n = min(chunk, total - c0)
            h = stacked[:, c0:c0 + n].reshape(n_seq * n, c.hidden).clone()
            for i in range(c.layers):
                self._prefill_layer(i, h, n_seq, start + c0)
        last = h.view(n_seq, -1, c.hidden)[:, -1]
        for b, d in enumerate(ds):
            d.h.copy_(last[b])
            d.position.fill_(start + total - 1)
            d.run_lm_head_select()
            d.run_token_store(advance=True)

    def run_decode_layers(self, trace: torch.Tensor | None = None) -> None:
        """Every sequence's layers in one persistent launch; ``trace`` (kernels.decode_layers_trace) records its
        phase timeline."""
        ds, c = self.decoders, self.decoders[0].config
        kernels.decode_layers_seqs([d.layer_table for d in ds], [d.h for d in ds], [d.position for d in ds],
                                   [d.layers_ws for d in ds], [d.status for d in ds], hidden=c.hidden, mlp=c.mlp,
                                   nh=c.heads, nk=c.kv_heads, d=c.head_dim, s_cap=ds[0].max_positions,
                                   eps=c.rms_eps, theta=c.rope_theta, trace=trace)

    def run_lm_heads(self) -> None:
        """Every sequence's final norm + LM head + per-block argmax: one launch that reads a Q4_K head once for
        all of them (bit-identical to each sequence's own), else one launch per sequence."""
        ds = self.decoders
        d0 = ds[0]
        shared = all(d._w("lm_head").data_ptr() == d0._w("lm_head").data_ptr()
                     and d._n("norm").data_ptr() == d0._n("norm").data_ptr() for d in ds)
        if shared and d0.types["lm_head"] == "q4_k" and d0.config.hidden in (1024, 4096):
            kernels.q4k_lm_head_argmax_partial_seqs([d.h for d in ds], d0._w("lm_head"),
                                                    [d.partial_scores for d in ds], [d.partial_tokens for d in ds],
                                                    norm_weight=d0._n("norm"), eps=d0.config.rms_eps)
        else:
            for d in ds:
                d._lm_head()

    def run_decode_embeds(self) -> None:
        """Every sequence's next token into its residual stream: one launch for a shared Q4_K embedding, else
        one per sequence."""
        ds = self.decoders
        d0 = ds[0]
        if d0.types["embed"] == "q4_k" and all(d._w("embed").data_ptr() == d0._w("embed").data_ptr() for d in ds):
            kernels.embedding_q4_k_seqs(d0._w("embed"), [d.next_token.view(-1) for d in ds], d0.config.hidden,
                                        [d.h for d in ds])
        else:
            for d in ds:
                d.run_decode_embed()

    def run_select_stores(self) -> None:
        """Every sequence's greedy select + token store + position advance: one launch when the sequences
        share the EOS policy and the generated capacity, else one per sequence."""
        ds = self.decoders
        d0 = ds[0]
        if all(d.stop_on_eos == d0.stop_on_eos and d.generated.numel() == d0.generated.numel() for d in ds):
            kernels.token_select_store_seqs([d.partial_scores for d in ds], [d.partial_tokens for d in ds], d0.eos,
                                            [d.next_token for d in ds], [d.done for d in ds],
                                            [d.generated for d in ds], [d.length for d in ds],
                                            [d.stopped for d in ds], stop_on_eos=d0.stop_on_eos,
                                            advance=[d.position for d in ds])
        else:
            for d in ds:
                d._select_store()

    def decode_step(self) -> None:
        self.run_decode_embeds()
        self.run_decode_layers()
        self.run_lm_heads()
        self.run_select_stores()

    def graph(self, steps: int) -> torch.cuda.CUDAGraph:
        """A graph of ``steps`` consecutive group decode steps (captured once per step count)."""
        if steps not in self._graphs:
            saved = [d._save_state() for d in self.decoders]
            dev = self.decoders[0].device
            side = torch.cuda.Stream(device=dev)
            side.wait_stream(torch.cuda.current_stream(dev))
            with torch.cuda.stream(side):
                self.decode_step()  # warm-up launch outside capture
            torch.cuda.current_stream(dev).wait_stream(side)
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                for _ in range(steps):
                    self.decode_step()
            for d, st in zip(self.decoders, saved):
                d._restore_state(st)
            self._graphs[steps] = g
        return self._graphs[steps]

    def run_steps(self, n: int, steps_per_graph: int = 8, use_graph: bool = True) -> None:
        if not use_graph:
            for _ in range(n):
                self.decode_step()
            return
        full, rest = divmod(n, steps_per_graph)
        if full:
            g = self.graph(steps_per_graph)
            for _ in range(full):
                g.replay()
        for _ in range(rest):
            self.decode_step()

    def finish(self, max_new_tokens: int, steps_per_graph: int = 8, use_graph: bool = True) -> list[list[int]]:
        """After every decoder's prefill (which stored its first token): the remaining tokens of all of them
        together; each sequence's generated ids."""
        for d in self.decoders:
            d._check_budget(int(d.position.item()), max_new_tokens)
        self.run_steps(max_new_tokens - 1, steps_per_graph=steps_per_graph, use_graph=use_graph)
        out = []
        for d in self.decoders:
            d.check_status()
            out.append(d.generated[:int(d.length.item())].tolist())
        return out
