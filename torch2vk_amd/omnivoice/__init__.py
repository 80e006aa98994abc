"""OmniVoice on libt2h: the acoustic decoder composed from the conv1d, conv_transpose1d, snake, embedding and
linear kernels (the LLM pass is Qwen3Decoder.forward_masked; the token loop is in kernels.omnivoice_*)."""
