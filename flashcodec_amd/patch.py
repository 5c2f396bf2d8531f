"""One-call hot patch that gives a HuggingFace causal LM a codec KV cache.

transformers routes every KV write and read through ``cache.update(k, v,
layer_idx)``, so handing the model a codec cache replaces its KV storage
without touching the model (flashcodec/patch.py:1-136).  Same public
functions and ``model._flashcodec`` record as the reference; the patch
itself is an ``_Injection`` object that owns everything it changed:

* ``apply_flash_codec(model, ...)`` installs entry points on the model
  instance that hand a fresh FlashCodecCache to ``generate`` (caching on by
  default) and to ``forward`` calls that ask for a cache, whenever the
  caller passes none; ``materialization_free=True`` also routes decode-step
  attention through the coefficient-domain kernels (patch_attention);
* ``remove_flash_codec(model)`` (alias ``undo_flash_codec``) puts back
  exactly what was there before.
"""

import functools
import warnings

from .cache import HAS_HF_CACHE, CodecKVCache, FlashCodecCache

__all__ = ["apply_flash_codec", "remove_flash_codec", "undo_flash_codec",
           "find_attention_modules"]

_CODEC_DEFAULTS = (("keep_freqs", 2), ("keep_ratio", 1.0), ("quant_bits", 0),
                   ("quant_group", 0), ("packed", False))


def find_attention_modules(model):
    """Modules with both k_proj and v_proj (standard KV projections)."""
    return [m for m in model.modules() if hasattr(m, "k_proj") and hasattr(m, "v_proj")]


class _Injection:
    """One model's patch: the cache recipe, the caches handed out so far and
    the entry points it replaced."""

    ENTRY_POINTS = ("generate", "forward")

    def __init__(self, model, mode, block_size, options):
        self.model = model
        self.mode, self.block_size = mode, block_size
        self.codec_kw = {name: options.get(name, default) for name, default in _CODEC_DEFAULTS}
        self.per_layer = options.get("per_layer")
        self.config = getattr(model, "config", None)
        self.caches = []
        # (bound original, whether it was an instance attribute of its own)
        self.saved = {name: (getattr(model, name), name in vars(model))
                      for name in self.ENTRY_POINTS}

    def new_cache(self):
        """A cache for one generation: per-layer from the model config when
        possible (hybrid models keep transformers' layers where attention is
        not full), else uniform; CodecKVCache without transformers."""
        cache = None
        if HAS_HF_CACHE and self.config is not None:
            try:
                cache = FlashCodecCache.from_config(self.config, mode=self.mode,
                                                    block_size=self.block_size,
                                                    per_layer=self.per_layer, **self.codec_kw)
            except Exception:
                cache = None
        if cache is None:
            kind = FlashCodecCache if HAS_HF_CACHE else CodecKVCache
            cache = kind(mode=self.mode, block_size=self.block_size, **self.codec_kw)
        self.caches.append(cache)
        return cache

    def _entry(self, name, wants_cache):
        original = self.saved[name][0]

        @functools.wraps(original)
        def entry(*args, **kw):
            if kw.get("past_key_values") is None and wants_cache(kw.get("use_cache")):
                kw["past_key_values"] = self.new_cache()
            return original(*args, **kw)
        return entry

    def install(self, materialization_free):
        model = self.model
        attention = find_attention_modules(model)
        # generate caches unless told not to; forward only when asked to
        model.generate = self._entry("generate", lambda use: use is None or bool(use))
        model.forward = self._entry("forward", lambda use: bool(use))
        wrapped = 0
        if materialization_free:
            from .patch_attention import apply_codec_attention
            wrapped = apply_codec_attention(model)
        model._flashcodec = {"mode": self.mode, "caches": self.caches,
                             "attention_modules": attention,
                             "codec_attention_modules": wrapped, "undo": self.uninstall}
        if not attention:
            warnings.warn("no attention module with k_proj/v_proj found — if the model uses a "
                          "non-standard KV interface, the patch may have no effect")

    def uninstall(self):
        from .patch_attention import remove_codec_attention
        model = self.model
        remove_codec_attention(model)
        for name, (original, own) in self.saved.items():
            if own:
                setattr(model, name, original)
            elif name in vars(model):
                delattr(model, name)      # the class's method shows through again
        model._flashcodec = None


def apply_flash_codec(model, mode="jpeg", block_size=8, materialization_free=False, **kwargs):
    """Give every cached ``generate`` / ``forward`` of `model` a codec KV
    cache (flashcodec/patch.py:63-117).

    mode="jpeg": kwargs keep_freqs (default 2), quant_bits (0 or 8);
    mode="png": kwarg keep_ratio (default 1.0); per_layer maps layer indices
    to codec overrides.  ``materialization_free=True`` also patches
    Llama/Qwen-style attention so decode steps attend on the stored rows.
    Returns the model; ``remove_flash_codec(model)`` undoes everything."""
    if getattr(model, "_flashcodec", None) is not None:
        warnings.warn("model is already patched with flashcodec, call remove_flash_codec first")
        return model
    _Injection(model, mode, block_size, kwargs).install(materialization_free)
    return model


def remove_flash_codec(model):
    """Undo apply_flash_codec (both entry points and any attention patch)."""
    record = getattr(model, "_flashcodec", None)
    if record is not None:
        record["undo"]()


undo_flash_codec = remove_flash_codec
