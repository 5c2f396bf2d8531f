"""Codec KV cache: per-stream device state, layer pairs, the duck-typed
multi-layer cache and the transformers-5.x Cache / DynamicLayer backends.

Behaviour and attribute layout follow flashcodec/cache.py:39-654 (callers
and tests read the buffers by name); the organisation is this build's own:

* ``_CodecStream`` (one K or V tensor of one layer, layout (B, H, S, D),
  codec axis -2) is device state only.  Its raw tail (< r tokens, full
  fidelity) is the first t rows of a preallocated (B, H, r, D) tail buffer,
  so a token append is one copy and a completed block is archived straight
  from that buffer.  The archive of complete blocks lives in buffers of
  ``capacity`` blocks (``_coeffs``/``_scales`` for jpeg,
  ``_deltas``/``_anchors`` for png) written in place by the archive kernels;
  ``_rec`` holds an append-only reconstruction that ``read()`` extends only
  by the blocks archived since the last read.
* Every structural change is device work of libflashcodec_amd.so: capacity
  growth and batch gathers (beam reorders, batch selection or expansion)
  are gathers of per-(row, head) byte prefixes (``fc_gather_segments``; in
  place for a same-size reorder, so a captured HIP graph can replay it), and
  a crop that cuts into the archive reconstructs the boundary block's kept
  tokens directly into the tail buffer.
* ``_KVPair`` holds the key and value streams of one layer (one codec); the
  multi-layer ``CodecKVCache`` and the transformers ``FlashCodecLayer`` /
  ``FlashCodecCache`` are thin shells over pairs.

Only complete blocks are archived, so future tokens never rewrite archived
bits (causal safety).
"""

from functools import partial

import torch

from . import _native as N
from .codecs import JPEGCodec, PNGCodec
from .codecs import jpeg as _jpeg
from .codecs import png as _png

try:  # transformers 5.x layer-container Cache
    from transformers.cache_utils import Cache as _HFCache
    from transformers.cache_utils import DynamicLayer as _HFDynamicLayer
    HAS_HF_CACHE = True
except Exception:  # transformers absent: CodecKVCache still works
    _HFCache = object
    _HFDynamicLayer = object
    HAS_HF_CACHE = False

_FIRST_CAPACITY = 16   # archive blocks of a stream's first allocation


def make_codec(mode="jpeg", block_size=8, keep_freqs=2, keep_ratio=1.0, quant_bits=0,
               quant_group=0, packed=False):
    """Codec instance from a mode name (flashcodec/cache.py:39-54); png keeps
    fp32 deltas on purpose and rejects quant_bits.  This build's extensions:
    quant_group=32 (jpeg with quant_bits=8) scales every 32 features of a
    coefficient row separately; packed=True (png with keep_ratio < 1) stores
    only the Top-M surviving deltas of each (block, feature) plus a mask
    word."""
    if mode == "png":
        if quant_bits or quant_group:
            raise ValueError("quant_bits is only supported for mode='jpeg' "
                             "(the png lossless tier must keep fp32 deltas)")
        return PNGCodec(block_size=block_size, keep_ratio=keep_ratio, packed=packed)
    if packed:
        raise ValueError("packed=True is a png option (Top-M delta packing)")
    if mode == "jpeg":
        return JPEGCodec(block_size=block_size, keep_freqs=keep_freqs, quant_bits=quant_bits,
                         quant_group=quant_group)
    raise ValueError(f"unknown mode: {mode!r} (expected 'jpeg' | 'png')")


def _capacity_for(blocks):
    """Archive capacity holding `blocks`: the first allocation's 16 blocks,
    doubled as often as needed (flashcodec/cache.py:106-121)."""
    cap = _FIRST_CAPACITY
    while cap < blocks:
        cap <<= 1
    return cap


def _gather(dst, src, idx, live_rows):
    """dst[b, h, :live_rows] = src[idx[b], h, :live_rows] on the device for
    (B, H, rows, ...) buffers whose (b, h) runs are contiguous; idx None is
    the identity (a verbatim prefix copy), dst is src for an in-place
    reorder."""
    if live_rows <= 0 or dst.shape[0] == 0 or dst.shape[1] == 0:
        return
    es = dst.element_size()
    seg = live_rows * src.stride(2) * es
    rc = N.lib().fc_gather_segments(
        dst.data_ptr(), dst.stride(0) * es, dst.stride(1) * es, src.data_ptr(),
        src.stride(0) * es, src.stride(1) * es, N.ptr(idx), dst.shape[0], src.shape[0],
        dst.shape[1], seg, N.stream_ptr(src.device))
    N.check(rc, "fc_gather_segments")


def _device_index(idx, device, batch):
    """Batch indices as a device int64 tensor.  Outside a graph capture they
    are checked on the host (the reference's index_select raises on a bad
    index; the gather kernel skips one)."""
    idx = torch.as_tensor(idx)
    if not torch.cuda.is_current_stream_capturing():
        host = idx.cpu()
        if host.numel() and (int(host.min()) < 0 or int(host.max()) >= batch):
            raise IndexError(f"batch index out of range for a cache of batch {batch}")
    return idx.to(device=device, dtype=torch.int64).contiguous()


class _CodecStream:
    """One (B, H, S, D) stream: raw tail + capacity-doubling archive + the
    memoised reconstruction (flashcodec/cache.py:57-325)."""

    _INITIAL_BLOCKS = _FIRST_CAPACITY

    def __init__(self, codec):
        self.codec = codec
        self.n_blocks = 0        # archived blocks
        self.n_archived = 0      # archived tokens (n_blocks * r)
        self.meta = None         # (B, H, D, element size)
        self.dtype = None        # stream dtype, restored by read()
        self._capacity = 0       # allocated archive blocks
        self._coeffs = self._scales = None     # jpeg archive
        self._deltas = self._anchors = None    # png archive
        self._packed = self._packed_mask = None  # packed png archive
        self._raw_buf = None     # (B, H, r, D) tail buffer in the stream dtype
        self._n_raw = 0          # tokens in the tail (t < r)
        self._tail_rows = None   # per-row (B, H, 1, D) views of the tail buffer
        self._tail_key = None    # token (shape, dtype, device) the fast append path serves
        self._rec = None         # (B, H, tokens, D) reconstruction, stream dtype
        self._rec_blocks = 0     # blocks reconstructed into _rec
        self._rec_capacity = 0   # tokens allocated in _rec

    # ------------------------------------------------------------ shape
    @property
    def block_size(self):
        return self.codec.block_size

    @property
    def seq_len(self):
        return self.n_archived + self._n_raw

    @property
    def raw(self):
        """Raw tail (B, H, t, D), 0 < t < r, or None (flashcodec/cache.py:
        72-88): a view of the tail buffer, valid until the tail next
        completes a block."""
        return self._raw_buf[:, :, :self._n_raw] if self._n_raw else None

    @raw.setter
    def raw(self, value):
        if value is None or value.shape[-2] == 0:
            self._n_raw = 0
            return
        t = value.shape[-2]
        if t >= self.block_size:
            raise ValueError(f"a raw tail holds fewer than block_size={self.block_size} tokens "
                             f"(got {t})")
        self._tail_buffer(value)[:, :, :t].copy_(value)
        self._n_raw = t

    def _tail_buffer(self, like):
        """The (B, H, r, D) tail buffer, reallocated when `like`'s batch,
        heads, width, dtype or device differ (the live rows move over)."""
        B, H, D = like.shape[0], like.shape[1], like.shape[-1]
        dtype = self.dtype if self.dtype is not None else like.dtype
        cur = self._raw_buf
        if (cur is not None and cur.shape[0] == B and cur.shape[1] == H and cur.shape[-1] == D
                and cur.dtype == dtype and cur.device == like.device):
            return cur
        buf = torch.empty((B, H, self.block_size, D), dtype=dtype, device=like.device)
        if self._n_raw and cur is not None and cur.shape == buf.shape:
            buf[:, :, :self._n_raw].copy_(cur[:, :, :self._n_raw])
        return self._adopt_tail(buf)

    def _adopt_tail(self, buf):
        self._raw_buf = buf
        self._tail_rows = [buf[:, :, t:t + 1] for t in range(self.block_size)]
        self._tail_key = None
        return buf

    # ------------------------------------------------------------ archive buffers
    def _archive_spec(self, cap, B, H, D):
        """(attribute, shape, dtype) of every archive buffer at capacity cap
        (the reference layout, flashcodec/cache.py:94-104)."""
        c = self.codec
        if c.name == "png" and c.packed:
            # packed Top-M deltas: slot values, mask words (kept steps and the
            # signs of the pruned ones), anchors
            return [("_packed", (B, H, cap, c.keep_m, D), torch.float32),
                    ("_anchors", (B, H, cap, D), self.dtype),
                    ("_packed_mask", (B, H, cap, D), torch.int32)]
        if c.name == "png":
            return [("_deltas", (B, H, cap, c.block_size - 1, D), torch.float32),
                    ("_anchors", (B, H, cap, D), self.dtype)]
        spec = [("_coeffs", (B, H, cap, c.keep_freqs, D),
                 torch.int8 if c.quantized else self.dtype)]
        if c.quantized:
            groups = D // c.quant_group if c.quant_group else 1
            spec.append(("_scales", (B, H, cap, c.keep_freqs, groups), torch.float32))
        return spec

    def _archive_tensors(self):
        if self.codec.name == "png" and self.codec.packed:
            return (self._packed, self._anchors, self._packed_mask)
        if self.codec.name == "png":
            return (self._deltas, self._anchors)
        return (self._coeffs, self._scales) if self.codec.quantized else (self._coeffs,)

    def _grow(self, need_blocks, like):
        """Make room for `need_blocks` archived blocks: new buffers of the
        next capacity, the archived prefix copied over on the device."""
        if need_blocks <= self._capacity:
            return
        cap = _capacity_for(need_blocks)
        B, H, D = like.shape[0], like.shape[1], like.shape[-1]
        for name, shape, dtype in self._archive_spec(cap, B, H, D):
            fresh = torch.empty(shape, dtype=dtype, device=like.device)
            old = getattr(self, name)
            if self.n_blocks and old is not None:
                _gather(fresh, old, None, self.n_blocks)
            setattr(self, name, fresh)
        self._capacity = cap

    def _archive(self, head):
        """Encode the complete blocks of head (B, H, m*r, D) into the
        archive at block offset n_blocks (flashcodec/cache.py:123-141)."""
        r = self.block_size
        m = head.shape[-2] // r
        if not m:
            return
        self._grow(self.n_blocks + m, head)
        if head.stride(-1) != 1:
            head = head.contiguous()
        c = self.codec
        if c.name == "png" and c.packed:
            _png.encode_packed_into(head, r, c.keep_m, self._packed, self._packed_mask,
                                    self._anchors, self._capacity, self.n_blocks, m, m * r)
        elif c.name == "png":
            _png.encode_into(head, r, c.keep_m, self._deltas, self._anchors, self._capacity,
                             self.n_blocks, m, m * r)
        else:
            if c.quant_group and head.shape[-1] % c.quant_group:
                raise ValueError(f"quant_group={c.quant_group} needs a head size that is a "
                                 f"multiple of it (got {head.shape[-1]})")
            _jpeg.encode_into(head, r, c.keep_freqs, c.quant_bits, self._coeffs, self._scales,
                              self._capacity, self.n_blocks, m, m * r,
                              group=getattr(c, "quant_group", 0))
        self.n_blocks += m

    def _reconstruct(self, first, count, out, out_len, token0=0):
        """Reconstruct archived blocks [first, first+count) into `out`
        (row 0 = token `token0`; tokens >= out_len are not written)."""
        c, r = self.codec, self.block_size
        like = self._archive_tensors()[0]
        B, H, D = like.shape[0], like.shape[1], like.shape[-1]
        if c.name == "png" and c.packed:
            _png.decode_packed_into(self._packed, self._packed_mask, self._anchors, B, H,
                                    self._capacity, first, count, D, r, c.keep_m, out, out_len,
                                    token0)
        elif c.name == "png":
            _png.decode_into(self._deltas, self._anchors, B, H, self._capacity, first, count, D,
                             r, out, out_len, token0)
        else:
            _jpeg.decode_into(self._coeffs, self._scales, B, H, self._capacity, first, count, D,
                              r, c.keep_freqs, out, out_len, token0, group=c.quant_group)

    # ------------------------------------------------------------ write
    def append(self, tokens):
        """Append (B, H, m, D) tokens (flashcodec/cache.py:143-159): every
        block they complete is archived now, the rest waits in the tail.
        The archived bits depend only on each block's r tokens, so whole
        blocks of the input are encoded straight from the input and a block
        completed by the tail from the tail buffer."""
        r = self.block_size
        t = self._n_raw
        if (t + 1 < r and self._tail_key is not None
                and self._tail_key == (tokens.shape, tokens.dtype, tokens.device)):
            self._tail_rows[t].copy_(tokens)       # one token into a checked buffer
            self._n_raw = t + 1
            return
        N.require_gpu(tokens)
        if self.meta is None:
            self.meta = (tokens.shape[0], tokens.shape[1], tokens.shape[-1],
                         tokens.element_size())
            self.dtype = tokens.dtype
        m = tokens.shape[-2]
        if not m:
            return
        buf = self._tail_buffer(tokens)
        if m == 1 and tokens.dtype == self.dtype:
            self._tail_key = (tokens.shape, tokens.dtype, tokens.device)
        if t + m < r:
            buf[:, :, t:t + m].copy_(tokens)
            self._n_raw = t + m
            return
        used = 0
        if t:
            used = r - t
            buf[:, :, t:].copy_(tokens[:, :, :used])
            self._archive(buf)
            self.n_archived += r
            self._n_raw = 0
        whole = (m - used) // r * r
        if whole:
            self._archive(tokens[:, :, used:used + whole])
            self.n_archived += whole
        left = m - used - whole
        if left:
            buf[:, :, :left].copy_(tokens[:, :, used + whole:])
        self._n_raw = left

    # ------------------------------------------------------------ read
    def _decode_pending(self):
        """Extend _rec by the blocks archived since the last read (append
        only: reconstructed tokens are never recomputed)."""
        done, total = self._rec_blocks, self.n_blocks
        if done >= total:
            return
        r = self.block_size
        like = self._archive_tensors()[0]
        if self._rec is None or self._rec.shape[-2] < total * r:
            tokens = max(total * r, 2 * self._rec_capacity, _FIRST_CAPACITY * r)
            rec = torch.empty((like.shape[0], like.shape[1], tokens, like.shape[-1]),
                              dtype=self.dtype, device=like.device)
            if self._rec is not None and done:
                _gather(rec, self._rec, None, done * r)
            self._rec, self._rec_capacity = rec, tokens
        self._reconstruct(done, total - done, self._rec, total * r)
        self._rec_blocks = total

    def discard_view(self):
        """Drop the reconstruction (read() rebuilds it on demand)."""
        self._rec, self._rec_blocks, self._rec_capacity = None, 0, 0

    def read(self):
        """Reconstructed (B, H, S, D) view in the stream dtype
        (flashcodec/cache.py:203-220): archived tokens from _rec (a view when
        the tail is empty) followed by the raw tail."""
        if not self.n_blocks:
            # a copy: the tail buffer's rows are rewritten once a block completes
            return None if not self._n_raw else self.raw.clone()
        self._decode_pending()
        view = self._rec[:, :, :self.n_archived]
        return view if not self._n_raw else torch.cat([view, self.raw], dim=-2)

    # ------------------------------------------------------------ structure
    def reset(self):
        """Forget the contents, keep the allocations."""
        self._n_raw = 0
        self.n_blocks = self.n_archived = self._rec_blocks = 0

    def crop(self, tokens_to_remove):
        """Drop trailing tokens (negative count, HF semantics;
        flashcodec/cache.py:230-257).  Archived blocks before the cut stay
        verbatim; when the cut falls inside the archive, the kept tokens of
        the boundary block are reconstructed straight into the tail buffer,
        so repeated crops add no loss."""
        if tokens_to_remove > 0:
            raise ValueError("crop only supports negative values (remove trailing tokens)")
        if not tokens_to_remove:
            return
        r = self.block_size
        keep = max(0, self.seq_len + tokens_to_remove)
        blocks, tail = divmod(keep, r)
        if blocks < self.n_blocks:
            if tail:
                buf = self._tail_buffer(self._archive_tensors()[0])
                self._reconstruct(blocks, 1, buf, keep, token0=blocks * r)
            self.n_blocks, self.n_archived = blocks, blocks * r
            self._rec_blocks = min(self._rec_blocks, blocks)
        self._n_raw = tail

    def select_batch(self, idx):
        """Gather batch rows (beam-search reorder, batch selection or
        expansion; flashcodec/cache.py:259-301).  A reorder that keeps the
        batch size gathers the archive and the tail in place (one kernel per
        buffer, no allocation); _rec is rebuilt in a new buffer because
        read() may have handed out views into the current one."""
        live = self._archive_tensors()[0] if self.n_blocks else self._raw_buf
        if live is None or (not self.n_blocks and not self._n_raw and self._rec is None):
            return
        B_old = live.shape[0]
        idx = _device_index(idx, live.device, B_old)
        B_new = idx.numel()
        same = B_new == B_old
        if self.n_blocks:
            if same:
                for t in self._archive_tensors():
                    _gather(t, t, idx, self.n_blocks)
            else:
                H, D = live.shape[1], live.shape[-1]
                for name, shape, dtype in self._archive_spec(self._capacity, B_new, H, D):
                    fresh = torch.empty(shape, dtype=dtype, device=live.device)
                    _gather(fresh, getattr(self, name), idx, self.n_blocks)
                    setattr(self, name, fresh)
        if self._raw_buf is not None:
            if same:
                _gather(self._raw_buf, self._raw_buf, idx, self._n_raw)
            else:
                old = self._raw_buf
                fresh = torch.empty((B_new,) + tuple(old.shape[1:]), dtype=old.dtype,
                                    device=old.device)
                _gather(fresh, old, idx, self._n_raw)
                self._adopt_tail(fresh)
        if self._rec is not None:
            old = self._rec
            self._rec = torch.empty((B_new,) + tuple(old.shape[1:]), dtype=old.dtype,
                                    device=old.device)
            _gather(self._rec, old, idx, self._rec_blocks * self.block_size)
        if self.meta is not None:
            self.meta = (B_new,) + self.meta[1:]

    def storage_bytes(self):
        """Bytes of the archived blocks and the raw tail (capacity slack and
        _rec excluded)."""
        total = 0
        if self.n_blocks:
            for t in self._archive_tensors():
                total += t.element_size() * t[:, :, :self.n_blocks].numel()
        if self._n_raw:
            total += self.raw.element_size() * self.raw.numel()
        return total


class _KVPair:
    """Key and value streams of one attention layer, sharing one codec."""

    def __init__(self, codec):
        self.codec = codec
        self.key = _CodecStream(codec)
        self.value = _CodecStream(codec)

    def streams(self):
        return self.key, self.value

    def append(self, key_states, value_states):
        self.key.append(key_states)
        self.value.append(value_states)

    def views(self):
        return self.key.read(), self.value.read()

    def crop(self, tokens_to_remove):
        for st in self.streams():
            st.crop(tokens_to_remove)

    def select_batch(self, idx):
        for st in self.streams():
            st.select_batch(idx)

    def reset(self):
        for st in self.streams():
            st.reset()

    def storage_bytes(self):
        return self.key.storage_bytes() + self.value.storage_bytes()


class CodecKVCache:
    """Multi-layer codec KV cache usable without transformers, duck-typed as
    an HF cache (flashcodec/cache.py:328-440)::

        cache = CodecKVCache(mode="jpeg", block_size=8, keep_freqs=2)
        k, v = cache.update(k_states, v_states, layer_idx=0)   # incremental
        k, v = cache.forward(k_seq, v_seq, layer_idx=0)        # full sequence
    """

    def __init__(self, mode="jpeg", block_size=8, keep_freqs=2, keep_ratio=1.0,
                 quant_bits=0, quant_group=0, packed=False):
        self.mode = mode
        self.codec = make_codec(mode, block_size, keep_freqs, keep_ratio, quant_bits=quant_bits,
                                quant_group=quant_group, packed=packed)
        self._pairs = {}     # layer index -> _KVPair

    def _pair(self, layer_idx):
        pair = self._pairs.get(layer_idx)
        if pair is None:
            pair = self._pairs[layer_idx] = _KVPair(self.codec)
        return pair

    def _selected(self, layer_idx):
        if layer_idx is None:
            return list(self._pairs.values())
        return [self._pairs[layer_idx]] if layer_idx in self._pairs else []

    @property
    def _keys(self):
        return {i: p.key for i, p in self._pairs.items()}

    @property
    def _values(self):
        return {i: p.value for i, p in self._pairs.items()}

    def update(self, key_states, value_states, layer_idx=0):
        """Append (B, H, m, D) and return the layer's reconstructed views."""
        pair = self._pair(layer_idx)
        pair.append(key_states, value_states)
        return pair.views()

    decode_step = update

    def forward(self, key_seq, value_seq, layer_idx=0):
        """Restart the layer with a whole sequence; returns its views."""
        self.reset(layer_idx)
        return self.update(key_seq, value_seq, layer_idx)

    def reset(self, layer_idx=None):
        if layer_idx is None:
            self._pairs.clear()
        else:
            self._pairs.pop(layer_idx, None)

    def crop(self, tokens_to_remove, layer_idx=None):
        for pair in self._selected(layer_idx):
            pair.crop(tokens_to_remove)

    def reorder_cache(self, beam_idx, layer_idx=None):
        for pair in self._selected(layer_idx):
            pair.select_batch(beam_idx)

    def _views_by_layer(self, which):
        top = max(self._pairs, default=-1)
        out = []
        for i in range(top + 1):
            pair = self._pairs.get(i)
            out.append(None if pair is None else getattr(pair, which).read())
        return out

    @property
    def key_cache(self):
        return self._views_by_layer("key")

    @property
    def value_cache(self):
        return self._views_by_layer("value")

    def get_seq_length(self, layer_idx=0):
        pair = self._pairs.get(layer_idx)
        return pair.key.seq_len if pair is not None else 0

    def get_max_length(self):
        return None

    def get_usable_length(self, new_seq_length, layer_idx=0):
        return self.get_seq_length(layer_idx)

    def storage_bytes(self, layer_idx=None):
        return sum(pair.storage_bytes() for pair in self._selected(layer_idx))

    def stats(self, layer_idx=0):
        pair = self._pairs.get(layer_idx)
        if pair is None or pair.key.meta is None:
            return {"tokens": 0, "archived": 0, "raw": 0, "storage_bytes": 0, "raw_bytes": 0}
        B, H, D, elem = pair.key.meta
        tokens, archived = pair.key.seq_len, pair.key.n_archived
        return {"tokens": tokens, "archived": archived, "raw": tokens - archived,
                "storage_bytes": pair.storage_bytes(),
                "raw_bytes": 2 * tokens * B * H * D * elem}

    def __repr__(self):
        return f"CodecKVCache(mode={self.mode!r}, codec={self.codec}, layers={sorted(self._pairs)})"


class FlashCodecLayer(_HFDynamicLayer):
    """transformers-5.x cache layer backed by a pair of codec streams;
    ``update`` returns the reconstructed causal KV
    (flashcodec/cache.py:446-544)."""

    def __init__(self, mode="jpeg", block_size=8, keep_freqs=2, keep_ratio=1.0, quant_bits=0,
                 quant_group=0, packed=False):
        super().__init__()
        self.mode = mode
        self.codec = make_codec(mode, block_size, keep_freqs, keep_ratio, quant_bits=quant_bits,
                                quant_group=quant_group, packed=packed)
        self._pair = _KVPair(self.codec)

    @property
    def _key_stream(self):
        return self._pair.key

    @_key_stream.setter
    def _key_stream(self, stream):
        self._pair.key = stream

    @property
    def _value_stream(self):
        return self._pair.value

    @_value_stream.setter
    def _value_stream(self, stream):
        self._pair.value = stream

    def lazy_initialization(self, key_states, value_states):
        self.dtype, self.device = key_states.dtype, key_states.device
        self.keys = torch.tensor([], dtype=self.dtype, device=self.device)
        self.values = torch.tensor([], dtype=self.dtype, device=self.device)
        self.is_initialized = True

    def update(self, key_states, value_states, *args, **kwargs):
        if not self.is_initialized:
            self.lazy_initialization(key_states, value_states)
        self._pair.append(key_states, value_states)
        self.keys, self.values = self._pair.views()
        return self.keys, self.values

    def _refresh_views(self):
        """Rebuild the attention-facing views after a structural change."""
        if not self.is_initialized:
            return
        if self._pair.key.seq_len:
            self.keys, self.values = self._pair.views()
        else:
            self.keys = torch.empty(0, dtype=self.dtype, device=self.device)
            self.values = torch.empty(0, dtype=self.dtype, device=self.device)

    def get_seq_length(self):
        return self._pair.key.seq_len

    def get_max_length(self):
        return -1

    def crop(self, tokens_to_remove):
        self._pair.crop(tokens_to_remove)
        self._refresh_views()

    def select_batch(self, idx):
        self._pair.select_batch(idx)
        self._refresh_views()

    def reorder_cache(self, beam_idx):
        self.select_batch(beam_idx)

    def batch_repeat_interleave(self, repeats):
        if self.is_initialized:
            rows = torch.arange(self._pair.key.meta[0], device=self.device)
            self.select_batch(rows.repeat_interleave(repeats))

    def batch_select_indices(self, indices):
        if self.is_initialized:
            self.select_batch(indices)

    def reset(self):
        self._pair.reset()
        super().reset()

    def offload(self):
        pass  # archives stay on the device

    def prefetch(self):
        pass

    def storage_bytes(self):
        return self._pair.storage_bytes()


def _layer_plan(config, per_layer, codec_cfg):
    """One (kind, kwargs) per decoder layer of a model config: codec layers
    for full attention (codec_cfg with the per_layer override of that
    index), transformers' own dynamic layer type for the others (hybrid
    models; flashcodec/cache.py:585-626)."""
    from transformers.cache_utils import get_layer_types_and_kwargs
    decoder = config.get_text_config(decoder=True) if hasattr(config, "get_text_config") \
        else config
    try:
        types, kwargs = get_layer_types_and_kwargs(decoder)
    except Exception:
        n = getattr(decoder, "num_hidden_layers", 1)
        types = list(getattr(decoder, "layer_types", None) or ["full_attention"] * n)
        kwargs = {}
    # one kwargs dict shared by every layer (transformers 5.15) or one per layer
    per_index = kwargs if isinstance(kwargs, (list, tuple)) else [kwargs] * len(types)
    overrides = per_layer or {}
    for i, (kind, kw) in enumerate(zip(types, per_index)):
        if kind == "full_attention":
            yield kind, {**codec_cfg, **overrides.get(i, {})}
        else:
            yield kind, kw


class FlashCodecCache(_HFCache):
    """transformers-5.x codec KV cache (flashcodec/cache.py:547-654)::

        cache = FlashCodecCache(mode="jpeg", block_size=8, keep_freqs=2)
        model.generate(input_ids, past_key_values=cache, use_cache=True)
    """

    def __init__(self, mode="jpeg", block_size=8, keep_freqs=2, keep_ratio=1.0, quant_bits=0,
                 quant_group=0, packed=False):
        if not HAS_HF_CACHE:
            raise ImportError("FlashCodecCache requires transformers 5.x; use CodecKVCache "
                              "when transformers is unavailable.")
        cfg = dict(mode=mode, block_size=block_size, keep_freqs=keep_freqs,
                   keep_ratio=keep_ratio, quant_bits=quant_bits)
        if quant_group:
            cfg["quant_group"] = quant_group
        if packed:
            cfg["packed"] = True
        super().__init__(layers=None, layer_class_to_replicate=partial(FlashCodecLayer, **cfg))
        self._remember(cfg)

    def _remember(self, cfg, **extra):
        self.mode = cfg["mode"]
        self.codec_cfg = {k: v for k, v in cfg.items() if k != "mode"}
        self.codec_cfg.update(extra)

    @property
    def _seen_tokens(self):
        return self.get_seq_length()

    @classmethod
    def from_config(cls, config, mode="jpeg", block_size=8, keep_freqs=2, keep_ratio=1.0,
                    quant_bits=0, per_layer=None, quant_group=0, packed=False):
        """Per-layer cache for a model config: codec layers where the model
        uses full attention (each optionally overridden through
        ``per_layer[index]``), transformers' own layers elsewhere."""
        from transformers.cache_utils import DYNAMIC_LAYER_TYPE_MAPPING
        cfg = dict(mode=mode, block_size=block_size, keep_freqs=keep_freqs,
                   keep_ratio=keep_ratio, quant_bits=quant_bits)
        if quant_group:
            cfg["quant_group"] = quant_group
        if packed:
            cfg["packed"] = True
        layers = [FlashCodecLayer(**kw) if kind == "full_attention"
                  else DYNAMIC_LAYER_TYPE_MAPPING[kind](**kw)
                  for kind, kw in _layer_plan(config, per_layer, cfg)]
        cache = cls.__new__(cls)
        _HFCache.__init__(cache, layers=layers, layer_class_to_replicate=None)
        cache._remember(cfg, per_layer=per_layer)
        return cache

    def codec_layer_indices(self):
        return [i for i, layer in enumerate(self.layers) if isinstance(layer, FlashCodecLayer)]

    def to_legacy_cache(self):
        return {i: (layer.keys, layer.values) for i, layer in enumerate(self.layers)}

    @classmethod
    def from_legacy_cache(cls, legacy, **cfg):
        cache = cls(**cfg)
        for i in sorted(legacy):
            cache.update(legacy[i][0], legacy[i][1], i)
        return cache

    def storage_bytes(self, layer_idx=None):
        chosen = self.layers if layer_idx is None else [self.layers[layer_idx]]
        return sum(layer.storage_bytes() for layer in chosen if isinstance(layer, FlashCodecLayer))
