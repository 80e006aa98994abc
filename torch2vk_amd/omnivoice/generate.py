"""OmniVoice's masked-generation loop (src/models/quantized_omnivoice/run.py:56-60,217-300) on this library:
each step embeds the conditional and unconditional sequences (OMNIVOICE_INPUT_EMBED_Q8_0_F32), runs the Qwen3
backbone under each sequence's attention mask (run_llm_forward), the Q6_K audio head (run_audio_head),
classifier-free-guidance scoring (OMNIVOICE_CFG_SCORE_F32) and unmasks the scheduled number of best
positions (OMNIVOICE_TOKEN_UPDATE_TOPK_F32)."""

from __future__ import annotations

import math

import numpy as np
import torch

from torch2vk_amd import kernels
from torch2vk_amd.qwen3.model import Qwen3Decoder

RNG_SEED = 0x1234ABCD  # run.py's seed of the Gumbel noise


def time_steps(t_start: float, t_end: float, num_step: int, t_shift: float) -> np.ndarray:
    """The shifted time grid of run.py:56-60: t' = s t / (1 + (s - 1) t) over num_step + 1 points."""
    t = np.linspace(t_start, t_end, num_step + 1, dtype=np.float64)
    return (t_shift * t / (1.0 + (t_shift - 1.0) * t)).astype(np.float32)


def unmask_schedule(total_mask: int, num_steps: int, t_shift: float = 0.1) -> list[int]:
    """Positions unmasked per step (run.py:224-234): ceil(total * dt) capped by what remains; the last step
    takes the remainder.  The product is float32, as the reference's int times a float32 grid difference is
    under numpy 2's promotion rules; in float64 some totals round across an integer (221 over 8 steps)."""
    t = time_steps(0.0, 1.0, num_steps, t_shift)
    rem, out = total_mask, []
    for s in range(num_steps):
        num = rem if s == num_steps - 1 else min(math.ceil(np.float32(total_mask) * (t[s + 1] - t[s])), rem)
        out.append(int(num))
        rem -= int(num)
    return out


class OmniVoiceGenerator:
    """State: batch_input_ids int64 [2, C, S] (row 0 conditional with the T target frames last, row 1
    unconditional with them first), batch_audio_mask [2, S], attention masks fp32 [2, S, S], tokens int64
    [C * T] (mask_id where undecided)."""

    def __init__(self, llm: Qwen3Decoder, text_w: torch.Tensor, audio_w: torch.Tensor, head_w: torch.Tensor, *,
                 codebooks: int, vocab: int, mask_id: int) -> None:
        self.llm, self.text_w, self.audio_w, self.head_w = llm, text_w, audio_w, head_w
        self.c, self.v, self.mask_id = codebooks, vocab, mask_id

    def logits(self, ids: torch.Tensor, audio_mask: torch.Tensor, attn_mask: torch.Tensor) -> torch.Tensor:
        """fp32 [2, S, C * V]: input embedding, the backbone under each row's mask, the Q6_K audio head."""
        hidden = kernels.omnivoice_input_embed_q8_0(self.text_w, self.audio_w, ids, audio_mask, self.v)
        s = int(ids.shape[2])
        out = torch.empty(2, s, self.c * self.v, dtype=torch.float32, device=ids.device)
        for b in range(2):
            h = self.llm.forward_masked(hidden[b], attn_mask[b])
            kernels.gemm(kernels.im2col_1d(h.view(1, s, -1), 1), self.head_w, "q6_k", out=out[b],
                         out_dtype=torch.float32)
        return out

    def generate(self, ids: torch.Tensor, audio_mask: torch.Tensor, attn_mask: torch.Tensor, tokens: torch.Tensor, *,
                 num_steps: int, guidance: float, layer_penalty: float, temperature: float, t_shift: float = 0.1,
                 seed: int = RNG_SEED, on_step=None) -> torch.Tensor:
        """Run the loop in place on ids and tokens; returns tokens [C * T]."""
        t_len = tokens.numel() // self.c
        for step, k in enumerate(unmask_schedule(tokens.numel(), num_steps, t_shift)):
            if k <= 0:
                continue  # nothing left to unmask: the reference skips the step (run.py:251-253)
            lg = self.logits(ids, audio_mask, attn_mask)
            ct, cs = kernels.omnivoice_cfg_score(lg, tokens, codebooks=self.c, targets=t_len, vocab=self.v,
                                                 guidance=guidance, layer_penalty=layer_penalty,
                                                 temperature=temperature, step=step, seed=seed, mask_id=self.mask_id)
            kernels.omnivoice_token_update_topk(ct, cs, tokens, ids, unmask_count=k)
            if on_step is not None:
                on_step(step, k, lg)
        return tokens
