"""One-line hot patch that makes a HuggingFace CausalLM use FlashCodecCache.

transformers routes every KV write/read through ``cache.update(k, v,
layer_idx)``, so swapping the cache object replaces the KV storage without
model surgery (flashcodec/patch.py:1-136):

* ``apply_flash_codec(model, ...)`` wraps ``model.generate`` and
  ``model.forward`` to inject a FlashCodecCache when a cache is requested and
  none is passed; ``materialization_free=True`` also routes decode-step
  attention through ``codec_decode_attention``;
* ``remove_flash_codec(model)`` restores both wrappers.
"""

import functools
import warnings

from .cache import HAS_HF_CACHE, CodecKVCache, FlashCodecCache

__all__ = ["apply_flash_codec", "remove_flash_codec", "undo_flash_codec",
           "find_attention_modules"]


def find_attention_modules(model):
    """Attention modules with k_proj and v_proj projections."""
    return [m for m in model.modules() if hasattr(m, "k_proj") and hasattr(m, "v_proj")]


def _cache_factory(mode, block_size, kwargs, sink, config=None):
    codec_kw = dict(keep_freqs=kwargs.get("keep_freqs", 2),
                    keep_ratio=kwargs.get("keep_ratio", 1.0),
                    quant_bits=kwargs.get("quant_bits", 0))
    per_layer = kwargs.get("per_layer")

    def factory():
        cache = None
        if HAS_HF_CACHE and config is not None:
            # hybrid models: only full-attention layers carry a codec
            try:
                cache = FlashCodecCache.from_config(config, mode=mode, block_size=block_size,
                                                    per_layer=per_layer, **codec_kw)
            except Exception:
                cache = None
        if cache is None:
            cache = (FlashCodecCache(mode=mode, block_size=block_size, **codec_kw)
                     if HAS_HF_CACHE else
                     CodecKVCache(mode=mode, block_size=block_size, **codec_kw))
        sink.append(cache)
        return cache

    return factory


def apply_flash_codec(model, mode="jpeg", block_size=8, materialization_free=False, **kwargs):
    """Inject a codec KV cache into every ``generate`` / cached ``forward`` of
    ``model`` (flashcodec/patch.py:63-117).

    mode="jpeg": kwargs keep_freqs (default 2), quant_bits (0 or 8);
    mode="png": kwarg keep_ratio (default 1.0); per_layer overrides per layer
    index.  ``materialization_free=True`` also patches Llama/Qwen-style
    attention forwards so decode steps attend on the stored rows.
    Returns the model; ``remove_flash_codec(model)`` undoes everything."""
    if getattr(model, "_flashcodec", None) is not None:
        warnings.warn("model is already patched with flashcodec, call remove_flash_codec first")
        return model
    attns = find_attention_modules(model)
    caches = []
    factory = _cache_factory(mode, block_size, kwargs, caches,
                             config=getattr(model, "config", None))
    base_generate, base_forward = model.generate, model.forward

    @functools.wraps(base_generate)
    def generate(*args, **kw):
        use_cache = kw.get("use_cache")
        if (use_cache is None or use_cache) and kw.get("past_key_values") is None:
            kw["past_key_values"] = factory()
        return base_generate(*args, **kw)

    @functools.wraps(base_forward)
    def forward(*args, **kw):
        if kw.get("use_cache") and kw.get("past_key_values") is None:
            kw["past_key_values"] = factory()
        return base_forward(*args, **kw)

    model.generate = generate
    model.forward = forward
    n_wrapped = 0
    if materialization_free:
        from .patch_attention import apply_codec_attention
        n_wrapped = apply_codec_attention(model)
    model._flashcodec = {"mode": mode, "caches": caches, "attention_modules": attns,
                         "codec_attention_modules": n_wrapped,
                         "undo": lambda: _restore(model, base_generate, base_forward)}
    if not attns:
        warnings.warn("no attention module with k_proj/v_proj found — if the model uses a "
                      "non-standard KV interface, the patch may have no effect")
    return model


def _restore(model, base_generate, base_forward):
    from .patch_attention import remove_codec_attention
    remove_codec_attention(model)
    model.generate = base_generate
    model.forward = base_forward
    model._flashcodec = None


def remove_flash_codec(model):
    """Undo apply_flash_codec (restores generate and forward)."""
    info = getattr(model, "_flashcodec", None)
    if info is not None:
        info["undo"]()


undo_flash_codec = remove_flash_codec
