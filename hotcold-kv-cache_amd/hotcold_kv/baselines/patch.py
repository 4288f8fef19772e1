"""LlamaAttention monkeypatch for the compression baselines
(src/hotcold_kv/baselines/patch.py:37-103).

The patched forward projects Q/K/V, applies RoPE, and hands prefill/decode to
the active PressCache's layer; decode attention runs on the gfx950 kernel.
Only one attention patch (this one or the hot/cold one) may be installed.
"""

import math

from transformers.models.llama import modeling_llama

from .cache import PressCacheLayer

ACTIVE_PRESS_CACHE = None
_ORIG = None


def set_active_press_cache(cache):
    """Register the PressCache the patched attention routes through."""
    global ACTIVE_PRESS_CACHE
    ACTIVE_PRESS_CACHE = cache


def uninstall_press_patch():
    global _ORIG
    if _ORIG is not None:
        modeling_llama.LlamaAttention.forward = _ORIG
        _ORIG = None


def install_press_patch():
    global _ORIG
    if _ORIG is not None:
        return
    _ORIG = modeling_llama.LlamaAttention.forward
    orig = _ORIG

    def patched_forward(self, hidden_states, position_embeddings=None, attention_mask=None, past_key_values=None,
                        **kwargs):
        if ACTIVE_PRESS_CACHE is None or past_key_values is None:
            return orig(self, hidden_states, position_embeddings=position_embeddings,
                        attention_mask=attention_mask, past_key_values=past_key_values, **kwargs)
        layer = past_key_values.layers[self.layer_idx]
        if not isinstance(layer, PressCacheLayer):
            return orig(self, hidden_states, position_embeddings=position_embeddings,
                        attention_mask=attention_mask, past_key_values=past_key_values, **kwargs)

        num_heads = int(self.config.num_attention_heads)
        num_kv_heads = int(getattr(self.config, "num_key_value_heads", num_heads))
        head_dim = int(self.head_dim) if hasattr(self, "head_dim") else int(self.config.hidden_size // num_heads)
        n_rep = num_heads // num_kv_heads
        scaling = 1.0 / math.sqrt(head_dim)
        bsz, q_len, _ = hidden_states.shape

        q = self.q_proj(hidden_states).view(bsz, q_len, num_heads, head_dim).transpose(1, 2)
        k = self.k_proj(hidden_states).view(bsz, q_len, num_kv_heads, head_dim).transpose(1, 2)
        v = self.v_proj(hidden_states).view(bsz, q_len, num_kv_heads, head_dim).transpose(1, 2)
        cos, sin = position_embeddings
        q_post, k_post = modeling_llama.apply_rotary_pos_emb(q, k, cos, sin)

        if layer.get_seq_length() == 0:
            attn_out = layer.prefill(q_post, k_post, v, n_rep, scaling)     # (B,Hq,T,D)
        else:
            if q_len != 1:
                raise NotImplementedError("multi-token forward on a compressed cache is not supported")
            attn_out = layer.decode(q_post, k_post, v, n_rep, scaling)      # (B,Hq,1,D)

        attn_out = attn_out.transpose(1, 2).contiguous().view(bsz, q_len, -1)
        return self.o_proj(attn_out), None

    modeling_llama.LlamaAttention.forward = patched_forward
