"""Route the attention of Llama/Qwen-style modules on codec layers through
the coefficient-domain kernels (flashcodec/patch_attention.py:1-151).

``apply_flash_codec`` swaps the cache, but transformers still attends on the
reconstructed view.  This patch replaces the forward of standard attention
modules (q_proj / k_proj / v_proj / o_proj, optional q_norm / k_norm, plain
or gated query projection).  On a codec layer the projections, norms and
RoPE run as usual; then
* a decode step (one query token) appends K/V to the codec streams and
  attends on the archive in one library call (``codec_decode_step``);
* a prefill (several query tokens) on int8 jpeg archives appends the
  prompt's K/V and attends causally on the archive's stored rows
  (``codec_prefill_attention``): no reconstructed view is ever built.  Other
  archives (png, unquantised jpeg) run the model's own attention on the
  view the cache returns, released as soon as that forward returns, so a
  prefill holds one layer's view at a time (the reference keeps every
  layer's until that layer's first decode step, patch_attention.py:90-94).
  ``set_prefill_on_archive(False)`` selects that path for every archive.

Guards (anything else calls the original forward): codec cache layer, eval
mode, ``position_embeddings`` given, no sliding window, a RoPE function in
the model's module, and a mask the kernels honour.  Decode steps take the
codec path at batch 1 whatever the mask (as the reference does,
patch_attention.py:52-61) or with no mask at all (transformers passes none
to SDPA-style attention when nothing is padded, so unpadded batches take it
too).  A prefill on the archive applies the plain causal mask only, so it
runs there when the mask is absent or is exactly that mask (no padded key
columns: eager-attention models pass it explicitly); a padded prompt runs
the original forward with its mask.
"""

import importlib

import torch

from .attention import codec_decode_step, codec_prefill_attention, prefill_supported
from .cache import FlashCodecLayer

_ROPE_CACHE = {}


def _rope_fn(module):
    """``apply_rotary_pos_emb`` of the modeling file that defines the module."""
    name = type(module).__module__
    if name not in _ROPE_CACHE:
        _ROPE_CACHE[name] = getattr(importlib.import_module(name), "apply_rotary_pos_emb", None)
    return _ROPE_CACHE[name]


def _codec_layer(module, past_key_values):
    layers = getattr(past_key_values, "layers", None)
    if layers is None:
        return None
    try:
        layer = layers[module.layer_idx]
    except (IndexError, TypeError):
        return None
    return layer if isinstance(layer, FlashCodecLayer) else None


def _release_view(layer):
    """Drop a codec layer's reconstructed view (the streams' _rec and the
    layer's references to it); the archives and tails stay."""
    for st in (layer._key_stream, layer._value_stream):
        if st._rec is not None:
            st.discard_view()
    layer.keys = layer.values = None


def _project(module, hidden_states, position_embeddings):
    """q (B, Hq, T, D), k, v (B, Hkv, T, D) after the projections, the
    optional q/k norms and RoPE, plus the output gate of gated (Qwen3.5-
    style) query projections; the sequence is fixed by the HF attention
    modules this wraps."""
    lead = hidden_states.shape[:-1]
    hd = module.head_dim
    width = module.o_proj.in_features
    qp = module.q_proj(hidden_states)
    gate = None
    if module.q_proj.out_features == 2 * width:
        q, gate = torch.chunk(qp.view(*lead, -1, 2 * hd), 2, dim=-1)
        gate = gate.reshape(*lead, -1)
    else:
        q = qp
    q = q.view(*lead, -1, hd)
    k = module.k_proj(hidden_states).view(*lead, -1, hd)
    v = module.v_proj(hidden_states).view(*lead, -1, hd).transpose(1, 2)
    if hasattr(module, "q_norm"):
        q = module.q_norm(q)
    if hasattr(module, "k_norm"):
        k = module.k_norm(k)
    cos, sin = position_embeddings
    q, k = _rope_fn(module)(q.transpose(1, 2), k.transpose(1, 2), cos, sin)
    return q, k, v, gate


def _finish(module, out, gate, lead):
    out = out.transpose(1, 2).reshape(*lead, -1).contiguous()
    if gate is not None:
        out = out * torch.sigmoid(gate)
    return module.o_proj(out), None


def _plain_causal(mask, T, total):
    """Whether `mask` lets query i of a T-token prefill (position
    total - T + i) see exactly the keys 0 .. its own position: None, a 2-D
    (batch, key) padding mask with every one of the `total` keys kept, or a
    4-D (batch, 1 or heads, T, keys) mask (bool: True attends; additive
    float: 0 attends) equal to the causal pattern over the first `total`
    keys.  Reads the mask back to the host (prefill only: decode steps never
    call it, so they stay capturable)."""
    if mask is None:
        return True
    if not torch.is_tensor(mask):
        return False                      # e.g. a flex-attention block mask
    if mask.dim() == 2:
        return mask.shape[-1] >= total and bool(mask[:, :total].bool().all())
    if mask.dim() != 4 or mask.shape[-2] != T or mask.shape[-1] < total:
        return False
    m = mask[..., :total]
    seen = m if m.dtype == torch.bool else m == 0
    keys = torch.arange(total, device=mask.device)
    last = torch.arange(total - T, total, device=mask.device)
    allowed = keys[None, :] <= last[:, None]
    return bool(torch.equal(seen, allowed.expand_as(seen)))


def _attention_forward(module, orig, hidden_states, position_embeddings=None,
                       attention_mask=None, past_key_values=None, **kwargs):
    layer = _codec_layer(module, past_key_values)
    T = hidden_states.shape[-2]
    codec_ok = (layer is not None
                and not module.training
                and position_embeddings is not None
                and getattr(module, "sliding_window", None) is None
                and _rope_fn(module) is not None)
    if codec_ok and T == 1:
        codec_ok = hidden_states.shape[0] == 1 or attention_mask is None
    if (codec_ok and T > 1 and _PREFILL["on"]
            and prefill_supported(layer.codec, hidden_states.dtype, module.head_dim)
            and _plain_causal(attention_mask, T, layer.get_seq_length() + T)):
        # prefill on the archive: append the prompt's K/V, attend without a view
        q, k, v, gate = _project(module, hidden_states, position_embeddings)
        if not layer.is_initialized:
            layer.lazy_initialization(k, v)
        _release_view(layer)
        layer._pair.append(k, v)
        out = codec_prefill_attention(q, layer._key_stream, layer._value_stream,
                                      scale=module.scaling)
        module._flashcodec_prefills = getattr(module, "_flashcodec_prefills", 0) + 1
        return _finish(module, out, gate, hidden_states.shape[:-1])
    if not (codec_ok and T == 1):
        out = orig(hidden_states, position_embeddings=position_embeddings,
                   attention_mask=attention_mask, past_key_values=past_key_values, **kwargs)
        if codec_ok and T > 1 and layer.is_initialized:
            _release_view(layer)  # prefill done: decode attends on the archive
        return out

    q, k, v, gate = _project(module, hidden_states, position_embeddings)
    if not layer.is_initialized:
        layer.lazy_initialization(k, v)
    # the prefill view is dead weight once decoding attends on the archive
    _release_view(layer)
    # append both tokens and attend in one library call (two appends and an
    # attention call in the reference, patch_attention.py:95-98)
    out = codec_decode_step(q, k, v, layer._key_stream, layer._value_stream,
                            scale=module.scaling)
    module._flashcodec_codec_steps = getattr(module, "_flashcodec_codec_steps", 0) + 1
    return _finish(module, out, gate, hidden_states.shape[:-1])


# Reconstruct-free prefill switch (on by default; off runs the reference's
# prefill on the materialised view, for comparisons).
_PREFILL = {"on": True}


def set_prefill_on_archive(enabled):
    """Choose how patched prefills attend: on the archive's stored rows
    (True, the default: no reconstructed view) or on the reconstructed view
    through the model's own attention (False, the reference's semantics).
    Returns the previous setting."""
    prev = _PREFILL["on"]
    _PREFILL["on"] = bool(enabled)
    return prev


def _supported(module):
    if not all(hasattr(module, a) for a in
               ("q_proj", "k_proj", "v_proj", "o_proj", "layer_idx", "head_dim")):
        return False
    width = module.o_proj.in_features
    if module.head_dim <= 0 or width % module.head_dim:
        return False
    return module.q_proj.out_features in (width, 2 * width)


def apply_codec_attention(model):
    """Patch every supported attention module; idempotent.  Returns the
    number of wrapped modules."""
    wrapped = 0
    for module in model.modules():
        if not _supported(module):
            continue
        if getattr(module, "_flashcodec_orig_forward", None) is None:
            orig = module.forward

            def forward(*args, _module=module, _orig=orig, **kw):
                return _attention_forward(_module, _orig, *args, **kw)

            module._flashcodec_orig_forward = orig
            module.forward = forward
        wrapped += 1
    return wrapped


def remove_codec_attention(model):
    """Restore the original forwards; returns how many were restored."""
    restored = 0
    for module in model.modules():
        orig = getattr(module, "_flashcodec_orig_forward", None)
        if orig is not None:
            module.forward = orig
            del module._flashcodec_orig_forward
            restored += 1
    return restored


def codec_attention_stats(model):
    """Number of attention modules currently wrapped."""
    return sum(1 for m in model.modules()
               if getattr(m, "_flashcodec_orig_forward", None) is not None)
