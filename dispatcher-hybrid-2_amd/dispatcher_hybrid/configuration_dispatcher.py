"""DispatcherConfig: shape and behaviour switches of the Dispatcher-Hybrid causal LM.

Same arguments, defaults and validation as the reference configuration
(reference dispatcher_hybrid/configuration_dispatcher.py:35-102), so configs and checkpoints written
for the reference load unchanged. The defaults describe the released 292M model: 18 layers, of which
layers 8 and 17 (1-indexed) are sliding-window (1024) attention and the other 16 are dyadic mixers
with log2(max_len) = 12 levels.
"""

import math

from transformers import PretrainedConfig


class DispatcherConfig(PretrainedConfig):
    """Config of a Dispatcher / sliding-window-attention hybrid causal LM.

    Args:
        vocab_size: vocabulary (GPT-2 BPE, 50257).
        d_model, num_heads, dim_feedforward, num_layers: trunk shape.
        max_len: context length, a power of two; the mixer has log2(max_len) levels.
        attn_layers: 1-indexed positions of the attention layers (empty: pure mixer).
        attn_window: attention window; 0 turns the attention slots into mixer layers.
        gate_bias_flat, gate_fbias_flat: initial admit / forget gate biases.
        doc_reset: mixer edges may not cross an `eot_token` (document boundary).
        tie_word_embeddings: the output head shares the input embedding.
    """

    model_type = "dispatcher-hybrid"
    keys_to_ignore_at_inference = ["past_key_values"]

    def __init__(self, vocab_size=50257, d_model=1024, num_heads=16, dim_feedforward=2816,
                 num_layers=18, max_len=4096, attn_layers=(8, 17), attn_window=1024,
                 gate_bias_flat=-2.0, gate_fbias_flat=2.0, doc_reset=True, eot_token=50256,
                 tie_word_embeddings=True, use_cache=False, bos_token_id=50256,
                 eos_token_id=50256, **kwargs):
        if max_len <= 0 or (max_len & (max_len - 1)) != 0:
            raise ValueError(f"max_len must be a power of two, got {max_len}")
        if d_model % num_heads != 0:
            raise ValueError("d_model must be divisible by num_heads")
        self.vocab_size = vocab_size
        self.d_model = d_model
        self.num_heads = num_heads
        self.dim_feedforward = dim_feedforward
        self.num_layers = num_layers
        self.max_len = max_len
        self.attn_layers = tuple(attn_layers)
        self.attn_window = attn_window
        self.gate_bias_flat = gate_bias_flat
        self.gate_fbias_flat = gate_fbias_flat
        self.doc_reset = doc_reset
        self.eot_token = eot_token
        self.use_cache = use_cache
        super().__init__(tie_word_embeddings=tie_word_embeddings, bos_token_id=bos_token_id,
                         eos_token_id=eos_token_id, **kwargs)

    @property
    def levels(self):
        """Mixer levels: lags 1, 2, ..., max_len / 2."""
        return int(math.log2(self.max_len))

    # generic names some transformers utilities look up
    @property
    def hidden_size(self):
        return self.d_model

    @property
    def num_attention_heads(self):
        return self.num_heads

    @property
    def num_hidden_layers(self):
        return self.num_layers

    @property
    def max_position_embeddings(self):
        return self.max_len
