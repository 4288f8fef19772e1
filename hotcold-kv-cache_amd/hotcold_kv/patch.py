"""LlamaAttention monkeypatch of the hot/cold engine (src/hotcold_kv/patch.py).

The patched forward keeps the reference's four-tensor split -- q_pre for the
cold search, q_post for attention and scoring, k_pre for the cold store,
k_post for the hot cache, V never rotated -- and its knobs, and moves the hot
path onto the gfx950 kernels:
  * cache update: in-place append into the fixed-capacity hot buffer, device
    compression (HotColdLayer);
  * inject: a staged retrieval is re-rotated to its original positions and
    written into the held slot of the hot buffer in one kernel
    (patch.py:241-270 did _rotate_k_with_pos + torch.cat every step);
  * decode attention: one launch over [held slot | hot rows]; the held-slot
    mask valid & (pos <= cur_pos) is evaluated on the device, so there is no
    .item() host sync (patch.py:243, 284).
Prefill attention is the prompt's own causal attention (torch SDPA), as in
the reference (patch.py:317-337).
"""

import math

import torch
import torch.nn.functional as F
from transformers.cache_utils import Cache
from transformers.models.llama import modeling_llama

from . import ops
from .cache import HotColdLayer
from .datatypes import _canon_kv_4d

ACTIVE_KVCTRL = None
ACTIVE_ROTARY_EMB = None  # model.model.rotary_emb


def set_active_kvctrl(kvctrl):
    global ACTIVE_KVCTRL
    ACTIVE_KVCTRL = kvctrl


def set_active_rotary_emb(rotary_emb_module):
    global ACTIVE_ROTARY_EMB
    ACTIVE_ROTARY_EMB = rotary_emb_module


def _rope_params(device):
    """(inv_freq fp32 on device, attention_scaling) of the active rotary module."""
    if ACTIVE_ROTARY_EMB is None:
        raise RuntimeError("ACTIVE_ROTARY_EMB is None. Call set_active_rotary_emb(model.model.rotary_emb).")
    inv = ACTIVE_ROTARY_EMB.inv_freq.to(device=device, dtype=torch.float32)
    return inv, float(getattr(ACTIVE_ROTARY_EMB, "attention_scaling", 1.0))


def _rotate_k_with_pos(k_pre, pos_ids, head_dim=None):
    """Re-RoPE pre-RoPE keys (B,Hk,R,D) to positions (B,R) or (B,Hk,R)
    (patch.py:94-102), on the device.  Returns (B,Hk,R,D) in k_pre's dtype
    (fp32 input gives fp32 output)."""
    k_pre = _canon_kv_4d(k_pre, "k_pre")
    B, Hk, R, D = k_pre.shape
    inv, scale = _rope_params(k_pre.device)
    pos = pos_ids.long()
    cos, sin = ops.rope_tables(pos.reshape(-1, R), inv, scale, k_pre.dtype)    # the rotary module's tables
    shape = (B, Hk, R, D // 2) if pos.dim() == 3 else (B, R, D // 2)
    out_k = torch.empty((B, Hk, R, D), dtype=k_pre.dtype, device=k_pre.device)
    out_v = torch.empty_like(out_k)
    ops.inject_rerope_tab(k_pre.float().contiguous(), torch.zeros_like(k_pre, dtype=torch.float32),
                          cos.reshape(shape).contiguous(), sin.reshape(shape).contiguous(), out_k, out_v)
    return out_k


def hotcold_attention(kvctrl, layer, li, q_pre, k_pre, v, q_post, k_post, pos_new, n_rep, scaling,
                      attention_mask=None, past_key_values=None):
    """One layer's attention on the hot/cold engine: the body of the patched
    LlamaAttention.forward between RoPE and o_proj (patch.py:152-337), on
    (B,H,T,D) q_pre/k_pre/v/q_post/k_post and absolute positions pos_new
    (B,T).  layer is the layer's HotColdLayer (None: plain cache in
    past_key_values, or none).  Returns (B,Hq,T,D).

    A one-token step whose append cannot trigger a compression appends inside
    the decode launch (HotColdLayer.append_attend); other steps append
    through HotColdLayer.update (which may compress and evict), then attend."""
    q_len = int(q_pre.shape[2])
    device = q_pre.device
    if kvctrl._rope is None and ACTIVE_ROTARY_EMB is not None:
        kvctrl.set_rope(ACTIVE_ROTARY_EMB.inv_freq, getattr(ACTIVE_ROTARY_EMB, "attention_scaling", 1.0))

    # retrieval pipeline (patch.py:164-172)
    if q_len == 1 or kvctrl.query_pool_size >= kvctrl.window_size:
        kvctrl.update_query_window(li, q_pre)
    kvctrl.maybe_launch_async_retrieval(li)
    kvctrl.maybe_prefetch_to_gpu(li, device=device, dtype=q_pre.dtype)

    fused = q_len == 1 and layer is not None and layer.decode_fusable()
    k_cur, v_cur = k_post, v
    if layer is not None:
        r = kvctrl.recent_size
        layer.set_last_query_post(q_post if q_len <= r else q_post[:, :, -r:, :].clone())
        if not fused:
            layer.update(key_states=k_post, value_states=v, layer_idx=li,
                         cache_kwargs={"pre_key_states": k_pre, "positions": pos_new})
    elif past_key_values is not None:
        past_key_values.update(k_post, v, li)

    if q_len > 1 and kvctrl.retrieve_after_prefill:
        kvctrl.launch_retrieval_now(li, q_pre[:, :, -kvctrl.query_pool_size:, :])
        kvctrl.maybe_prefetch_to_gpu(li, device=device, dtype=q_pre.dtype)

    kvctrl.last_injected_len = 0

    if q_len == 1 and layer is not None:
        injected = None
        rr = kvctrl.poll_staged_gpu(li)
        if rr.ready:
            kbuf, vbuf = layer.buf.held_storage()
            R = int(rr.k_pre.shape[2])
            cos_t, sin_t = rr.cos, rr.sin
            if cos_t is None:
                # searched before the rotary parameters were known, so no
                # tables travelled with the rows: build them here from the
                # staged positions as the rotary module does, so the held keys
                # are apply_rotary_pos_emb's bits as with shipped tables
                # (without a rotary module this raises, as patch.py:76-78)
                inv, ascale = _rope_params(device) if kvctrl._rope is None else \
                    (kvctrl._rope[0].to(device), kvctrl._rope[1])
                cos, sin = ops.rope_tables(rr.pos.reshape(-1, R), inv, ascale, kbuf.dtype)
                B, Hk, _, D = rr.k_pre.shape
                shape = (B, Hk, R, D // 2) if rr.pos.dim() == 3 else (B, R, D // 2)
                cos_t, sin_t = cos.reshape(shape).contiguous(), sin.reshape(shape).contiguous()
                kvctrl.dbg["rope_rows_direct"] += 1
            ops.inject_rerope_tab(rr.k_pre, rr.v, cos_t, sin_t, kbuf, vbuf)
            kvctrl.staged_consumed(li)
            injected = (rr.pos, rr.valid, R)
        held = kvctrl.resolve_held(li, injected)
        if fused:
            out = layer.append_attend(q_post, k_post, v, k_pre, pos_new, scaling, held)
            kvctrl.dbg["triton_decode_calls"] += 1
            return out                                                    # (B,Hq,1,D)
        if held is not None:
            pos_h, valid_h, R = held
            k_att, v_att = layer.buf.attended(with_held=True)
            k_att = k_att[:, :, layer.buf.held - R:]
            v_att = v_att[:, :, layer.buf.held - R:]
            out = ops.decode_attention(q_post, k_att, v_att, scaling, held_len=R, held_pos=pos_h,
                                       held_valid=valid_h, cur_pos=pos_new[0, -1:])
        else:
            k_att, v_att = layer.buf.attended(with_held=False)
            out = ops.decode_attention(q_post, k_att, v_att, scaling)
        kvctrl.dbg["triton_decode_calls"] += 1
        return out.unsqueeze(2)                                           # (B,Hq,1,D)
    if q_len == 1:
        # no hot/cold layer: attend over this step's cache entry only
        return ops.decode_attention(q_post, k_cur, v_cur, scaling).unsqueeze(2)
    kvctrl.dbg["triton_prefill_fallback"] += 1
    prev = layer.get_seq_length() - q_len if layer is not None else 0
    if prev > 0:
        raise NotImplementedError("multi-token forward on a non-empty hot cache (chunked prefill) "
                                  "is not supported by the hot/cold patch")
    k_rep = modeling_llama.repeat_kv(k_cur, n_rep) if n_rep > 1 else k_cur
    v_rep = modeling_llama.repeat_kv(v_cur, n_rep) if n_rep > 1 else v_cur
    return F.scaled_dot_product_attention(q_post, k_rep, v_rep, attn_mask=attention_mask,
                                          dropout_p=0.0, is_causal=attention_mask is None)


_ORIG = None


def uninstall_monkeypatch():
    global _ORIG
    if _ORIG is not None:
        modeling_llama.LlamaAttention.forward = _ORIG
        _ORIG = None


def install_monkeypatch(enable_debug: bool = True):
    global _ORIG
    if _ORIG is not None:
        return
    _ORIG = modeling_llama.LlamaAttention.forward
    orig = _ORIG

    def patched_forward(self, hidden_states, position_embeddings=None, attention_mask=None, past_key_values=None,
                        **kwargs):
        kvctrl = ACTIVE_KVCTRL
        if kvctrl is None:
            return orig(self, hidden_states, position_embeddings=position_embeddings,
                        attention_mask=attention_mask, past_key_values=past_key_values, **kwargs)

        num_heads = int(self.config.num_attention_heads)
        num_kv_heads = int(getattr(self.config, "num_key_value_heads", num_heads))
        head_dim = int(self.head_dim) if hasattr(self, "head_dim") else int(self.config.hidden_size // num_heads)
        bsz, q_len, _ = hidden_states.shape
        device = hidden_states.device
        li = self.layer_idx

        q_pre = self.q_proj(hidden_states).view(bsz, q_len, num_heads, head_dim).transpose(1, 2)
        k_pre = self.k_proj(hidden_states).view(bsz, q_len, num_kv_heads, head_dim).transpose(1, 2)
        v = self.v_proj(hidden_states).view(bsz, q_len, num_kv_heads, head_dim).transpose(1, 2)
        kvctrl._lazy_init(k_pre, n_layers=int(self.config.num_hidden_layers))

        cos, sin = position_embeddings
        q_post, k_post = modeling_llama.apply_rotary_pos_emb(q_pre, k_pre, cos, sin)

        layer = None
        if isinstance(past_key_values, Cache) and isinstance(past_key_values.layers[li], HotColdLayer):
            layer = past_key_values.layers[li]
        prev = layer.get_seq_length() if layer is not None else 0

        # absolute positions of this step's tokens
        cache_position = kwargs.get("cache_position")
        position_ids = kwargs.get("position_ids")
        if cache_position is not None and int(cache_position.numel()) == q_len:
            pos_new = cache_position.reshape(1, -1).expand(bsz, -1).to(device=device, dtype=torch.long)
        elif position_ids is not None and position_ids.shape[-1] == q_len:
            pos_new = position_ids.reshape(-1, q_len).expand(bsz, -1).to(device=device, dtype=torch.long)
        else:
            pos_new = torch.arange(prev, prev + q_len, device=device, dtype=torch.long).unsqueeze(0).expand(bsz, -1)
        pos_new = pos_new.contiguous()

        attn_out = hotcold_attention(kvctrl, layer, li, q_pre, k_pre, v, q_post, k_post, pos_new,
                                     num_heads // num_kv_heads, 1.0 / math.sqrt(head_dim),
                                     attention_mask=attention_mask,
                                     past_key_values=past_key_values if layer is None else None)
        attn_out = attn_out.transpose(1, 2).contiguous().view(bsz, q_len, -1)
        attn_out = self.o_proj(attn_out)

        if enable_debug and kvctrl._inited and li == 0 and (kvctrl.step_count[0] % 50 == 0):
            ready_rate = kvctrl.dbg["prefetch_ready"] / max(1, kvctrl.dbg["prefetch_launched"])
            hot0 = past_key_values.layers[0].hot_length() if layer is not None else -1
            print("[DBG]", "step0", kvctrl.step_count[0], "hot0", hot0, "cold0", kvctrl.cold_size(0),
                  "ready_rate", round(ready_rate, 3))
        return attn_out, None

    modeling_llama.LlamaAttention.forward = patched_forward
