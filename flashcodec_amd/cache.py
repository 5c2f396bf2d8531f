"""Codec KV cache: per-stream state, the duck-typed multi-layer cache and the
transformers-5.x Cache/DynamicLayer backends.

Mirrors flashcodec/cache.py:39-654.  A stream (one K or V tensor of one
layer, layout (B, H, S, D), codec axis -2) keeps
  * a raw tail of < r tokens at full fidelity (``raw``: a view of the first
    t rows of a preallocated (B, H, r, D) tail buffer, so appending a token
    is one copy and a completed block is archived straight from the buffer),
  * an archive of complete blocks in capacity-doubling device buffers that
    are written in place by the archive kernels (``_coeffs``/``_scales`` for
    jpeg, ``_deltas``/``_anchors`` for png; reference layout, cache.py:94-104),
  * an append-only reconstructed view ``_rec`` that ``read()`` extends with
    the reconstruction kernels only for blocks archived since the last read.
Only complete blocks are archived, so future tokens never rewrite archived
bits (causal safety).  All arithmetic is in libflashcodec_amd.so; the tensor
bookkeeping (capacity growth, batch gathers, tail concatenation) uses
PyTorch device operations.
"""

import torch

from . import _native as N
from .codecs import JPEGCodec, PNGCodec
from .codecs import jpeg as _jpeg
from .codecs import png as _png

try:  # transformers 5.x layer-container Cache
    from functools import partial

    from transformers.cache_utils import Cache as _HFCache
    from transformers.cache_utils import DynamicLayer as _HFDynamicLayer
    HAS_HF_CACHE = True
except Exception:  # transformers absent: CodecKVCache still works
    _HFCache = object
    _HFDynamicLayer = object
    HAS_HF_CACHE = False


def make_codec(mode="jpeg", block_size=8, keep_freqs=2, keep_ratio=1.0, quant_bits=0):
    """Codec instance from a mode name (cache.py:39-54).  png keeps fp32
    deltas on purpose and rejects quant_bits."""
    if mode == "jpeg":
        return JPEGCodec(block_size=block_size, keep_freqs=keep_freqs, quant_bits=quant_bits)
    if mode == "png":
        if quant_bits:
            raise ValueError("quant_bits is only supported for mode='jpeg' "
                             "(the png lossless tier must keep fp32 deltas)")
        return PNGCodec(block_size=block_size, keep_ratio=keep_ratio)
    raise ValueError(f"unknown mode: {mode!r} (expected 'jpeg' | 'png')")


class _CodecStream:
    """One (B, H, S, D) stream: raw tail + capacity-doubling archive + the
    memoised reconstruction (cache.py:57-325)."""

    _INITIAL_BLOCKS = 16

    def __init__(self, codec):
        self.codec = codec
        self._raw_buf = None     # (B, H, r, D) tail buffer in the stream dtype
        self._n_raw = 0          # tokens in the tail (t < r)
        self._tail_rows = None   # per-row (B, H, 1, D) views of the tail buffer
        self._tail_key = None    # (shape, dtype, device) the tail buffer was checked for
        self.n_archived = 0      # archived tokens
        self.n_blocks = 0        # archived blocks
        self.meta = None         # (B, H, D, element size)
        self.dtype = None        # stream dtype, restored by read()
        self._capacity = 0       # allocated archive blocks
        self._coeffs = None      # jpeg: (B, H, cap, k, D) int8 or stream dtype
        self._scales = None      # jpeg int8: (B, H, cap, k, 1) fp32
        self._deltas = None      # png: (B, H, cap, r-1, D) fp32
        self._anchors = None     # png: (B, H, cap, D) stream dtype
        self._rec = None         # (B, H, rec_capacity, D) stream dtype
        self._rec_blocks = 0     # blocks already reconstructed into _rec
        self._rec_capacity = 0   # tokens allocated in _rec

    @property
    def block_size(self):
        return self.codec.block_size

    @property
    def raw(self):
        """Raw tail (B, H, t, D) with 0 < t < r, or None (cache.py:72-88): a
        view of the tail buffer, valid until the tail next completes a
        block."""
        if self._n_raw == 0:
            return None
        return self._raw_buf[:, :, :self._n_raw]

    @raw.setter
    def raw(self, value):
        if value is None or value.shape[-2] == 0:
            self._n_raw = 0
            return
        t = value.shape[-2]
        if t >= self.block_size:
            raise ValueError(f"a raw tail holds fewer than block_size={self.block_size} tokens "
                             f"(got {t})")
        self._tail_buffer(value)
        self._raw_buf[:, :, :t].copy_(value)
        self._n_raw = t

    def _tail_buffer(self, like):
        """The (B, H, r, D) tail buffer, (re)allocated to match `like`."""
        buf = self._raw_buf
        B, H, D = like.shape[0], like.shape[1], like.shape[-1]
        dtype = self.dtype if self.dtype is not None else like.dtype
        if (buf is None or buf.shape[0] != B or buf.shape[1] != H or buf.shape[-1] != D
                or buf.dtype != dtype or buf.device != like.device):
            old = self._raw_buf
            buf = torch.empty((B, H, self.block_size, D), dtype=dtype, device=like.device)
            if self._n_raw and old is not None and old.shape == buf.shape:
                buf[:, :, :self._n_raw].copy_(old[:, :, :self._n_raw])
            self._raw_buf = buf
            self._tail_rows = [buf[:, :, t:t + 1] for t in range(self.block_size)]
            self._tail_key = None
        return buf

    @property
    def seq_len(self):
        return self.n_archived + self._n_raw

    # ------------------------------------------------------------ storage
    def _archive_spec(self, cap, B, H, D):
        """(attribute, shape, dtype) of each archive buffer at capacity cap."""
        c = self.codec
        if c.name == "jpeg":
            if c.quantized:
                return [("_coeffs", (B, H, cap, c.keep_freqs, D), torch.int8),
                        ("_scales", (B, H, cap, c.keep_freqs, 1), torch.float32)]
            return [("_coeffs", (B, H, cap, c.keep_freqs, D), self.dtype)]
        return [("_deltas", (B, H, cap, c.block_size - 1, D), torch.float32),
                ("_anchors", (B, H, cap, D), self.dtype)]

    def _archive_tensors(self):
        if self.codec.name == "jpeg":
            return (self._coeffs, self._scales) if self.codec.quantized else (self._coeffs,)
        return (self._deltas, self._anchors)

    def _grow(self, need_blocks, like):
        """Double the capacity (from 16 blocks) until need_blocks fit, keeping
        the archived prefix verbatim."""
        if need_blocks <= self._capacity:
            return
        cap = max(self._INITIAL_BLOCKS, 1)
        while cap < need_blocks:
            cap *= 2
        B, H, D = like.shape[0], like.shape[1], like.shape[-1]
        for name, shape, dtype in self._archive_spec(cap, B, H, D):
            buf = torch.empty(shape, dtype=dtype, device=like.device)
            if self.n_blocks:
                buf[:, :, :self.n_blocks].copy_(getattr(self, name)[:, :, :self.n_blocks])
            setattr(self, name, buf)
        self._capacity = cap

    def _archive(self, head):
        """Encode the complete blocks of head (B, H, m*r, D) straight into the
        archive buffers at block offset n_blocks."""
        r = self.block_size
        m = head.shape[-2] // r
        if m == 0:
            return
        self._grow(self.n_blocks + m, head)
        if head.stride(-1) != 1:
            head = head.contiguous()
        c = self.codec
        if c.name == "jpeg":
            _jpeg.encode_into(head, r, c.keep_freqs, c.quant_bits, self._coeffs, self._scales,
                              self._capacity, self.n_blocks, m, m * r)
        else:
            _png.encode_into(head, r, c.keep_m, self._deltas, self._anchors, self._capacity,
                             self.n_blocks, m, m * r)
        self.n_blocks += m

    # ------------------------------------------------------------ write
    def append(self, tokens):
        """Append (B, H, m, D) tokens; every block completed by them is
        archived at once (cache.py:143-159).  Tokens that do not complete a
        block are copied into the tail buffer; a block completed by the tail
        is archived from the tail buffer, whole blocks of the input straight
        from the input (the archived bits depend only on each block's r
        tokens, so they equal the reference's cat-then-archive)."""
        r = self.block_size
        t = self._n_raw
        if (t + 1 < r and self._tail_key is not None
                and self._tail_key == (tokens.shape, tokens.dtype, tokens.device)):
            # one token for a buffer already checked against this token shape
            self._tail_rows[t].copy_(tokens)
            self._n_raw = t + 1
            return
        N.require_gpu(tokens)
        if self.meta is None:
            self.meta = (tokens.shape[0], tokens.shape[1], tokens.shape[-1],
                         tokens.element_size())
            self.dtype = tokens.dtype
        m = tokens.shape[-2]
        if m == 0:
            return
        if m == 1 and tokens.dtype == self.dtype:
            self._tail_buffer(tokens)
            self._tail_key = (tokens.shape, tokens.dtype, tokens.device)
        if t + m < r:
            # the tail grows: one copy (the common decode step)
            self._tail_buffer(tokens)[:, :, t:t + m].copy_(tokens)
            self._n_raw = t + m
            return
        pos = 0
        if t:
            # the tail completes a block
            buf = self._tail_buffer(tokens)
            pos = r - t
            buf[:, :, t:].copy_(tokens[:, :, :pos])
            self._archive(buf)
            self.n_archived += r
            self._n_raw = 0
        full = ((m - pos) // r) * r
        if full:
            self._archive(tokens[:, :, pos:pos + full])
            self.n_archived += full
        rem = m - pos - full
        if rem:
            self._tail_buffer(tokens)[:, :, :rem].copy_(tokens[:, :, pos + full:])
        self._n_raw = rem

    # ------------------------------------------------------------ read
    def _decode_pending(self):
        """Reconstruct the blocks archived since the last read into _rec
        (append-only, so earlier tokens are never recomputed)."""
        a, b = self._rec_blocks, self.n_blocks
        if a >= b:
            return
        r = self.block_size
        like = self._coeffs if self.codec.name == "jpeg" else self._deltas
        B, H, D = like.shape[0], like.shape[1], like.shape[-1]
        if self._rec is None or self._rec.shape[-2] < b * r:
            cap = max(b * r, self._rec_capacity * 2, self._INITIAL_BLOCKS * r)
            rec = torch.empty((B, H, cap, D), dtype=self.dtype, device=like.device)
            if self._rec is not None and a:
                rec[:, :, :a * r].copy_(self._rec[:, :, :a * r])
            self._rec, self._rec_capacity = rec, cap
        c = self.codec
        if c.name == "jpeg":
            _jpeg.decode_into(self._coeffs, self._scales, B, H, self._capacity, a, b - a, D, r,
                              c.keep_freqs, self._rec, b * r)
        else:
            _png.decode_into(self._deltas, self._anchors, B, H, self._capacity, a, b - a, D, r,
                             self._rec, b * r)
        self._rec_blocks = b

    def discard_view(self):
        """Drop the reconstructed view (rebuilt on demand by read())."""
        self._rec = None
        self._rec_blocks = 0
        self._rec_capacity = 0

    def read(self):
        """Reconstructed (B, H, S, D) view in the stream dtype: archived
        tokens from _rec (a view when there is no raw tail) followed by the
        raw tail (cache.py:203-220)."""
        if self.n_blocks == 0:
            # a copy: the tail buffer's rows are rewritten once a block completes
            return None if self.raw is None else self.raw.clone()
        self._decode_pending()
        view = self._rec[:, :, :self.n_archived]
        if self.raw is not None:
            view = torch.cat([view, self.raw], dim=-2)
        return view

    # ------------------------------------------------------------ structure
    def reset(self):
        """Forget the contents, keep the allocated capacity."""
        self.raw = None
        self.n_archived = 0
        self.n_blocks = 0
        self._rec_blocks = 0

    def crop(self, tokens_to_remove):
        """Drop trailing tokens (negative count, HF semantics).  Archived blocks
        stay verbatim; the partial block at the new end comes back as a raw
        tail taken from the reconstruction, so repeated crops add no loss
        (cache.py:230-257)."""
        if tokens_to_remove > 0:
            raise ValueError("crop only supports negative values (remove trailing tokens)")
        if tokens_to_remove == 0:
            return
        r = self.block_size
        keep = max(0, self.seq_len - abs(tokens_to_remove))
        keep_blocks, tail = divmod(keep, r)
        if keep_blocks < self.n_blocks:
            self._decode_pending()
            self.n_blocks = keep_blocks
            self.n_archived = keep_blocks * r
            self._rec_blocks = min(self._rec_blocks, keep_blocks)
            self.raw = self._rec[:, :, keep_blocks * r:keep, :].clone() if tail else None
        else:
            self._n_raw = tail      # the first `tail` rows of the tail buffer stay

    def select_batch(self, idx):
        """Gather batch rows (beam-search reorder, batch expansion)
        (cache.py:259-301)."""
        if self.raw is None and self.n_blocks == 0 and self._rec is None:
            return
        like = self.raw if self.raw is not None else self._archive_tensors()[0]
        idx = idx.to(like.device)
        r = self.block_size
        n = self.n_blocks
        if idx.numel() == like.shape[0]:
            # same batch size: archives are gathered in place; _rec is
            # replaced because read() may have handed out views into it
            if self.raw is not None:
                self.raw = self.raw.index_select(0, idx)
            if n:
                for t in self._archive_tensors():
                    t[:, :, :n] = t[:, :, :n].index_select(0, idx)
            if self._rec is not None and self._rec_blocks:
                done = self._rec_blocks * r
                rec = torch.empty_like(self._rec)
                rec[:, :, :done] = self._rec[:, :, :done].index_select(0, idx)
                self._rec = rec
            return
        B, H, D = idx.numel(), like.shape[1], like.shape[-1]
        for name, shape, dtype in self._archive_spec(self._capacity, B, H, D):
            old = getattr(self, name)
            buf = torch.empty(shape, dtype=dtype, device=like.device)
            if n:
                buf[:, :, :n] = old[:, :, :n].index_select(0, idx)
            setattr(self, name, buf)
        if self._rec is not None:
            rec = torch.empty((B, H, self._rec_capacity, D), dtype=self._rec.dtype,
                              device=like.device)
            if self._rec_blocks:
                done = self._rec_blocks * r
                rec[:, :, :done] = self._rec[:, :, :done].index_select(0, idx)
            self._rec = rec
        if self.raw is not None:
            self.raw = self.raw.index_select(0, idx)
        if self.meta is not None:
            self.meta = (B,) + self.meta[1:]

    def storage_bytes(self):
        """Bytes of the archived region plus the raw tail (capacity slack and
        _rec excluded)."""
        total = 0
        if self.n_blocks:
            for t in self._archive_tensors():
                total += t[:, :, :self.n_blocks].numel() * t.element_size()
        if self.raw is not None:
            total += self.raw.numel() * self.raw.element_size()
        return total


class CodecKVCache:
    """Multi-layer codec KV cache usable without transformers, duck-typed as
    an HF cache (cache.py:328-440)::

        cache = CodecKVCache(mode="jpeg", block_size=8, keep_freqs=2)
        k, v = cache.update(k_states, v_states, layer_idx=0)   # incremental
        k, v = cache.forward(k_seq, v_seq, layer_idx=0)        # full sequence
    """

    def __init__(self, mode="jpeg", block_size=8, keep_freqs=2, keep_ratio=1.0,
                 quant_bits=0):
        self.mode = mode
        self.codec = make_codec(mode, block_size, keep_freqs, keep_ratio, quant_bits=quant_bits)
        self._keys = {}
        self._values = {}

    def _stream(self, store, layer_idx):
        if layer_idx not in store:
            store[layer_idx] = _CodecStream(self.codec)
        return store[layer_idx]

    def update(self, key_states, value_states, layer_idx=0):
        """Append (B, H, m, D) and return the layer's reconstructed views."""
        ks = self._stream(self._keys, layer_idx)
        vs = self._stream(self._values, layer_idx)
        ks.append(key_states)
        vs.append(value_states)
        return ks.read(), vs.read()

    decode_step = update

    def forward(self, key_seq, value_seq, layer_idx=0):
        """Reset the layer, archive the whole sequence, return the views."""
        self.reset(layer_idx)
        return self.update(key_seq, value_seq, layer_idx)

    def reset(self, layer_idx=None):
        if layer_idx is None:
            self._keys.clear()
            self._values.clear()
        else:
            self._keys.pop(layer_idx, None)
            self._values.pop(layer_idx, None)

    def _each(self, layer_idx):
        for store in (self._keys, self._values):
            for i, st in store.items():
                if layer_idx is None or i == layer_idx:
                    yield st

    def crop(self, tokens_to_remove, layer_idx=None):
        for st in self._each(layer_idx):
            st.crop(tokens_to_remove)

    def reorder_cache(self, beam_idx, layer_idx=None):
        for st in self._each(layer_idx):
            st.select_batch(beam_idx)

    @property
    def key_cache(self):
        top = max(self._keys, default=-1)
        return [self._keys[i].read() if i in self._keys else None for i in range(top + 1)]

    @property
    def value_cache(self):
        top = max(self._values, default=-1)
        return [self._values[i].read() if i in self._values else None for i in range(top + 1)]

    def get_seq_length(self, layer_idx=0):
        st = self._keys.get(layer_idx)
        return 0 if st is None else st.seq_len

    def get_max_length(self):
        return None

    def get_usable_length(self, new_seq_length, layer_idx=0):
        return self.get_seq_length(layer_idx)

    def storage_bytes(self, layer_idx=None):
        layers = ([layer_idx] if layer_idx is not None
                  else sorted(set(self._keys) | set(self._values)))
        total = 0
        for i in layers:
            for store in (self._keys, self._values):
                if i in store:
                    total += store[i].storage_bytes()
        return total

    def stats(self, layer_idx=0):
        ks = self._keys.get(layer_idx)
        if ks is None or ks.meta is None:
            return {"tokens": 0, "archived": 0, "raw": 0, "storage_bytes": 0, "raw_bytes": 0}
        B, H, D, elem = ks.meta
        tokens = ks.seq_len
        return {"tokens": tokens, "archived": ks.n_archived, "raw": tokens - ks.n_archived,
                "storage_bytes": self.storage_bytes(layer_idx),
                "raw_bytes": tokens * B * H * D * elem * 2}

    def __repr__(self):
        return (f"CodecKVCache(mode={self.mode!r}, codec={self.codec}, "
                f"layers={sorted(set(self._keys) | set(self._values))})")


class FlashCodecLayer(_HFDynamicLayer):
    """transformers-5.x cache layer backed by two codec streams; ``update``
    returns the reconstructed causal KV (cache.py:446-544)."""

    def __init__(self, mode="jpeg", block_size=8, keep_freqs=2, keep_ratio=1.0, quant_bits=0):
        super().__init__()
        self.mode = mode
        self.codec = make_codec(mode, block_size, keep_freqs, keep_ratio, quant_bits=quant_bits)
        self._key_stream = _CodecStream(self.codec)
        self._value_stream = _CodecStream(self.codec)

    def lazy_initialization(self, key_states, value_states):
        self.dtype, self.device = key_states.dtype, key_states.device
        self.keys = torch.tensor([], dtype=self.dtype, device=self.device)
        self.values = torch.tensor([], dtype=self.dtype, device=self.device)
        self.is_initialized = True

    def update(self, key_states, value_states, *args, **kwargs):
        if not self.is_initialized:
            self.lazy_initialization(key_states, value_states)
        self._key_stream.append(key_states)
        self._value_stream.append(value_states)
        self.keys = self._key_stream.read()
        self.values = self._value_stream.read()
        return self.keys, self.values

    def get_seq_length(self):
        return self._key_stream.seq_len

    def get_max_length(self):
        return -1

    def crop(self, tokens_to_remove):
        self._key_stream.crop(tokens_to_remove)
        self._value_stream.crop(tokens_to_remove)
        self._rebuild_views()

    def reorder_cache(self, beam_idx):
        self.select_batch(beam_idx)

    def batch_repeat_interleave(self, repeats):
        if not self.is_initialized:
            return
        idx = torch.arange(self._key_stream.meta[0], device=self.device)
        self.select_batch(idx.repeat_interleave(repeats))

    def batch_select_indices(self, indices):
        if not self.is_initialized:
            return
        self.select_batch(indices)

    def select_batch(self, idx):
        self._key_stream.select_batch(idx)
        self._value_stream.select_batch(idx)
        self._rebuild_views()

    def _rebuild_views(self):
        if not self.is_initialized:
            return
        if self._key_stream.seq_len > 0:
            self.keys = self._key_stream.read()
            self.values = self._value_stream.read()
        else:
            self.keys = torch.empty(0, dtype=self.dtype, device=self.device)
            self.values = torch.empty(0, dtype=self.dtype, device=self.device)

    def reset(self):
        self._key_stream.reset()
        self._value_stream.reset()
        super().reset()

    def offload(self):
        pass  # archives stay on the device

    def prefetch(self):
        pass

    def storage_bytes(self):
        return self._key_stream.storage_bytes() + self._value_stream.storage_bytes()


class FlashCodecCache(_HFCache):
    """transformers-5.x codec KV cache (cache.py:547-654)::

        cache = FlashCodecCache(mode="jpeg", block_size=8, keep_freqs=2)
        model.generate(input_ids, past_key_values=cache, use_cache=True)
    """

    def __init__(self, mode="jpeg", block_size=8, keep_freqs=2, keep_ratio=1.0, quant_bits=0):
        if not HAS_HF_CACHE:
            raise ImportError("FlashCodecCache requires transformers 5.x; use CodecKVCache "
                              "when transformers is unavailable.")
        super().__init__(layers=None, layer_class_to_replicate=partial(
            FlashCodecLayer, mode=mode, block_size=block_size, keep_freqs=keep_freqs,
            keep_ratio=keep_ratio, quant_bits=quant_bits))
        self.mode = mode
        self.codec_cfg = dict(block_size=block_size, keep_freqs=keep_freqs,
                              keep_ratio=keep_ratio, quant_bits=quant_bits)

    @property
    def _seen_tokens(self):
        return self.get_seq_length()

    @classmethod
    def from_config(cls, config, mode="jpeg", block_size=8, keep_freqs=2, keep_ratio=1.0,
                    quant_bits=0, per_layer=None):
        """Per-layer cache from a model config: full-attention layers get a codec
        layer (optionally overridden per index through ``per_layer``), other
        layer types keep transformers' own dynamic layer (cache.py:585-626)."""
        from transformers.cache_utils import DYNAMIC_LAYER_TYPE_MAPPING, \
            get_layer_types_and_kwargs
        decoder = (config.get_text_config(decoder=True)
                   if hasattr(config, "get_text_config") else config)
        try:
            layer_types, layer_kwargs = get_layer_types_and_kwargs(decoder)
        except Exception:
            n = getattr(decoder, "num_hidden_layers", 1)
            layer_types = list(getattr(decoder, "layer_types", None) or ["full_attention"] * n)
            layer_kwargs = {}
        # transformers returns one kwargs dict shared by every layer (5.15) or
        # one dict per layer (later releases)
        if isinstance(layer_kwargs, dict):
            layer_kwargs = [layer_kwargs] * len(layer_types)
        per_layer = per_layer or {}
        base = dict(mode=mode, block_size=block_size, keep_freqs=keep_freqs,
                    keep_ratio=keep_ratio, quant_bits=quant_bits)
        layers = []
        for idx, (ltype, lkw) in enumerate(zip(layer_types, layer_kwargs)):
            if ltype == "full_attention":
                layers.append(FlashCodecLayer(**{**base, **per_layer.get(idx, {})}))
            else:
                layers.append(DYNAMIC_LAYER_TYPE_MAPPING[ltype](**lkw))
        obj = cls.__new__(cls)
        _HFCache.__init__(obj, layers=layers, layer_class_to_replicate=None)
        obj.mode = mode
        obj.codec_cfg = dict(block_size=block_size, keep_freqs=keep_freqs,
                             keep_ratio=keep_ratio, quant_bits=quant_bits, per_layer=per_layer)
        return obj

    def codec_layer_indices(self):
        return [i for i, layer in enumerate(self.layers) if isinstance(layer, FlashCodecLayer)]

    def to_legacy_cache(self):
        return {i: (layer.keys, layer.values) for i, layer in enumerate(self.layers)}

    @classmethod
    def from_legacy_cache(cls, legacy, **cfg):
        cache = cls(**cfg)
        for layer_idx in sorted(legacy):
            k, v = legacy[layer_idx]
            cache.update(k, v, layer_idx)
        return cache

    def storage_bytes(self, layer_idx=None):
        layers = self.layers if layer_idx is None else [self.layers[layer_idx]]
        return sum(layer.storage_bytes() for layer in layers if isinstance(layer, FlashCodecLayer))
