"""CPU oracle for the torch2vk quantized Qwen3 hot path.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, as the checker.  The shipped package
``torch2vk_amd`` never imports it and fails loudly without its HIP library.

Parity status of each oracle function (what pins it):

* quantize_q8_0      - hand-derived known-answer blocks + closed-form bounds.
* quantize_q4_k      - lattice known-answer superblocks (exact recovery of
                       planted codes), agreement of three independent reference
                       decoders, error bounds, special cases.
* quantize_q6_k      - lattice known-answer superblocks, the K6/K26 word
                       decoder, error bounds, special cases.
* dequant_*          - the independent numpy decoders in quant.py.
* reference.*        - textbook formulas checked against torch SDPA and
                       transformers' Qwen3 (random-init, no download).
* GPU-bit level of the reference GLSL (packHalf2x16 rounding, contraction,
  GLSL round() ties): parity unpinned; pinned to this IEEE restatement.
"""

from oracle.quant import (  # noqa: F401
    build,
    decode_q4_k_embedding_style,
    decode_q4_k_gemm_style,
    decode_q4_k_gemv_style,
    decode_q6_k_codes,
    decode_q8_0_codes,
    dequant_q4_k,
    dequant_q6_k,
    dequant_q8_0,
    f16_bits_to_f32,
    f32_to_f16_bits,
    q4_k_values_from_codes,
    quantize_q4_k,
    quantize_q6_k,
    quantize_q8_0,
)
