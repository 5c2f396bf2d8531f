"""Materialisation-free decode attention on the codec archive.

Both codecs are linear along the token axis: an archived block of r tokens
is A @ S with S its s stored rows and A (r x s) the synthesis matrix (jpeg:
the DCT basis transposed; png: tril(1) over anchor + deltas).  For one query
token the scores are (q . S^T) A^T and the output (prob A) S, so the (S, D)
reconstruction never exists (flashcodec/attention.py:1-27).

`codec_decode_attention` keeps the reference signature
(flashcodec/attention.py:64) and runs the split-K decode attention of
libflashcodec_amd.so: one launch whose workgroups walk the archived blocks
(every kv head's rows read once per group of up to sixteen query heads) and
whose last workgroup per head group merges the split partials with the raw
tail.
"""

import ctypes

import torch

from . import _native as N
from .codecs import dct_basis
from .codecs.jpeg import device_basis as dct_basis_device

_A_CACHE = {}
_WORKSPACES = {}


def block_basis(codec, block_size, device=None, dtype=torch.float32):
    """Synthesis matrix A (r, s) of an archived block (attention.py:35-42)."""
    r = block_size
    if codec.name == "jpeg":
        return dct_basis(r, codec.keep_freqs, device=device, dtype=dtype).t()
    return torch.tril(torch.ones(r, r, dtype=dtype, device=device))


def _device_A(codec, r, device):
    device = torch.device(device)
    key = (codec.name, r, getattr(codec, "keep_freqs", 0), device.type, device.index)
    A = _A_CACHE.get(key)
    if A is None:
        A = block_basis(codec, r, dtype=torch.float32).contiguous().to(device)
        _A_CACHE[key] = A
    return A


def workspace(device, nbytes):
    """Workspace of the decode attention for the current stream of `device`,
    at least `nbytes` long.  Zero-filled when created: its arrival counters
    must start at zero, and every call returns them to zero, so the calls of
    one stream (which run in order) share it.  Calls on other streams get
    their own."""
    device = torch.device(device)
    key = (device.index, N.stream_ptr(device))
    ws = _WORKSPACES.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = torch.zeros(nbytes, dtype=torch.uint8, device=device)
        _WORKSPACES[key] = ws
    return ws


def _jpeg_kind(codec):
    """Store kind of a jpeg codec's archive for the decode attention."""
    if not codec.quantized:
        return N.STORE_JPEG_FP
    return N.STORE_JPEG_I8G if codec.quant_group else N.STORE_JPEG_I8


def _store_kind(codec):
    """(store kind, stored rows per block) of a codec's archive for the
    decode attention: jpeg k rows; png r rows (anchor + deltas), packed png
    keep_m value slots."""
    if codec.name == "jpeg":
        return _jpeg_kind(codec), codec.keep_freqs
    if codec.packed:
        return N.STORE_PNG_PACKED, codec.keep_m
    return N.STORE_PNG, codec.block_size


FUSED_MERGE_MAX_SPLITS = 64   # the matrix-core pass merges in-kernel up to this many splits


def launches_per_call(store_kind, n_splits):
    """Kernel launches of one fc_decode_attention call over archived blocks:
    one when the split pass merges its own partials (the vector-ALU pass
    always; the matrix-core pass up to FUSED_MERGE_MAX_SPLITS splits), else
    the split pass plus the merge pass."""
    if store_kind == N.STORE_JPEG_I8 and N.lib().fc_get_attention_pass() != N.PASS_VECTOR:
        return 1 if n_splits <= FUSED_MERGE_MAX_SPLITS else 2
    return 1


def _view(stream, keep):
    """fc_stream_view of a stream; tensors it points into are added to `keep`."""
    v = N.StreamView()
    c = stream.codec
    if stream.n_blocks:
        if c.name == "jpeg":
            v.rows = stream._coeffs.data_ptr()
            v.scales = stream._scales.data_ptr() if c.quantized else None
        elif c.packed:
            v.rows = stream._packed.data_ptr()
            v.anchors = stream._anchors.data_ptr()
            v.masks = stream._packed_mask.data_ptr()
        else:
            v.rows = stream._deltas.data_ptr()
            v.anchors = stream._anchors.data_ptr()
        v.cap = stream._capacity
    if stream._n_raw:
        # the raw tail is the first _n_raw rows of the (B, H, r, D) tail buffer
        raw = stream._raw_buf
        keep.append(raw)
        v.raw = raw.data_ptr()
        v.raw_sb, v.raw_sh, v.raw_st = raw.stride(0), raw.stride(1), raw.stride(2)
    return v


def _triton_refuses(query, ks, vs, D):
    """Why impl="triton" raises in the reference for this call, or None.
    The reference tries its Triton path for jpeg stores only (png stores go
    to the torch path whatever `impl` says, flashcodec/attention.py:91) and
    raises when that path returns None for them
    (flashcodec/triton_attention.py:154-173, attention.py:96-99)."""
    if ks.codec.name != "jpeg":
        return None
    if not query.is_cuda:
        return "the query is not on a GPU"
    if vs.codec.name != "jpeg":
        return "key and value codecs differ"
    if ks.n_blocks == 0:
        return "an empty archive"
    if D > 256:
        return f"head size {D} > 256"
    return None


def codec_decode_attention(query, key_stream, value_stream, scale=None, impl="auto",
                           _n_splits=None):
    """Attention of one new query token against a codec archive without
    materialising the reconstructed KV.

    Args:
        query: (B, Hq, 1, D) query of the current step.
        key_stream, value_stream: ``_CodecStream`` instances of one layer.
        scale: attention scale (default ``D ** -0.5``).
        impl: the reference's implementation selector
            (flashcodec/attention.py:64-99).  Every value computes on this
            build's HIP kernels (there is no other implementation); they keep
            the reference's error behaviour: ``"triton"`` raises RuntimeError
            for the jpeg cases the reference's Triton path does not support
            (an empty archive, D > 256, a query off the GPU), while
            ``"auto"``, ``"torch"`` (the reference's portable path) and any
            other value run every case.
    Returns:
        (B, Hq, 1, D) attention output in the query dtype.

    GQA: query head hq attends kv head hq // (Hq / Hkv).  Raises ValueError
    for more than one query token (prefill attends the materialised view).
    ``_n_splits`` overrides the split-K count (testing and tuning only).
    """
    B, Hq, Sq, D = query.shape
    if Sq != 1:
        raise ValueError("codec_decode_attention only supports a single query token "
                         f"(got Sq={Sq}); prefill should use the materialized view")
    if impl == "triton":
        why = _triton_refuses(query, key_stream, value_stream, D)
        if why is not None:
            raise RuntimeError("triton implementation does not support this case "
                               f"({why}; see codec_decode_attention_triton)")
    scale = D ** -0.5 if scale is None else float(scale)
    ks, vs = key_stream, value_stream
    if ks.codec.name != vs.codec.name:
        raise ValueError("key and value streams must use the same codec")
    nb = ks.n_blocks
    if vs.n_blocks != nb or vs.n_archived != ks.n_archived:
        raise ValueError("key and value streams hold different token counts")
    n_raw = ks._n_raw
    if vs._n_raw != n_raw:
        raise ValueError("key and value streams hold different token counts")
    if nb == 0 and n_raw == 0:
        return torch.zeros_like(query)                   # empty cache
    N.require_gpu(query)
    like = ks._raw_buf if nb == 0 else ks._archive_tensors()[0]
    N.require_gpu(like)
    Hkv = like.shape[1]
    assert Hq % Hkv == 0, f"query heads ({Hq}) must be a multiple of kv heads ({Hkv})"
    if like.shape[0] != B:
        raise ValueError(f"batch mismatch: query {B}, cache {like.shape[0]}")

    c = ks.codec
    r = ks.block_size
    kind, s = _store_kind(c)
    q = query if query.stride(-1) == 1 else query.contiguous()
    out = torch.empty_like(q)
    dev = q.device
    L = N.lib()
    n_splits = L.fc_attention_splits(kind, N.dtype_code(ks.dtype), N.dtype_code(q.dtype), s, nb,
                                     B, Hkv, Hq // Hkv, D, N.num_cus(dev))
    if _n_splits is not None and nb:
        # split count override (tests / tuning); trimmed to non-empty splits
        per = -(-nb // max(1, int(_n_splits)))
        n_splits = -(-nb // per)
    ws = None
    if n_splits:
        ws = workspace(dev, L.fc_attention_workspace_bytes(B, Hq, D, n_splits))
    A = _device_A(c, r, dev) if nb else None
    keep = []
    kv, vv = _view(ks, keep), _view(vs, keep)
    rc = L.fc_decode_attention(
        q.data_ptr(), N.dtype_code(q.dtype), q.stride(0), q.stride(1), B, Hq, Hkv, D, kind,
        N.dtype_code(ks.dtype), r, s, nb, kv, vv, n_raw, N.ptr(A), scale, out.data_ptr(),
        out.stride(0), out.stride(1), N.ptr(ws), n_splits, N.stream_ptr(dev))
    N.check(rc, "fc_decode_attention")
    return out


def prefill_supported(codec, dtype, head_dim):
    """Whether codec_prefill_attention runs streams of `codec` with queries
    of `dtype` and head size `head_dim`: int8 jpeg archives (one scale per
    row or per 32 features) with 1 / 2 / 4 kept frequencies, fp16 / bf16
    queries, head size 64 / 128 / 256."""
    return (codec.name == "jpeg" and codec.quantized
            and codec.keep_freqs in (1, 2, 4)
            and dtype in (torch.float16, torch.bfloat16) and head_dim in (64, 128, 256))


def codec_prefill_attention(query, key_stream, value_stream, scale=None):
    """Causal attention of the newest Sq cached tokens' queries over the
    whole cache, on the archive's stored rows (no reconstructed view).

    query (B, Hq, Sq, D) holds the queries of the last Sq tokens of the
    streams (positions seq_len - Sq .. seq_len - 1); token i attends every
    cached token up to its own position: archived blocks through the codec's
    synthesis matrix in the coefficient domain, raw-tail tokens at full
    precision.  Returns (B, Hq, Sq, D) in the query dtype.  This build's
    replacement for the reference's prefill on the materialised view
    (flashcodec/attention.py:24-26, flashcodec/patch_attention.py:58-61);
    int8 jpeg streams only (prefill_supported)."""
    ks, vs = key_stream, value_stream
    B, Hq, Sq, D = query.shape
    if not (prefill_supported(ks.codec, query.dtype, D) and _same_codec(ks.codec, vs.codec)):
        raise NotImplementedError("codec_prefill_attention runs int8 jpeg archives with "
                                  "fp16/bf16 queries, D in (64, 128, 256), keep_freqs in (1, 2, 4)")
    N.require_gpu(query)
    if ks.seq_len != vs.seq_len or ks.n_blocks != vs.n_blocks or ks.meta is None:
        raise ValueError("key and value streams hold different token counts")
    if Sq > ks.seq_len:
        raise ValueError(f"{Sq} query tokens but {ks.seq_len} cached tokens: the queries are "
                         "the newest cached tokens' (append their keys and values first)")
    Hkv = ks.meta[1]
    assert Hq % Hkv == 0, f"query heads ({Hq}) must be a multiple of kv heads ({Hkv})"
    c = ks.codec
    r = c.block_size
    scale = D ** -0.5 if scale is None else float(scale)
    q = query if query.stride(-1) == 1 else query.contiguous()
    if (q.data_ptr() % 16) or any(x % 8 for x in q.stride()[:3]):
        q = q.contiguous()
    out = torch.empty((B, Hq, Sq, D), dtype=q.dtype, device=q.device)
    keep = []
    kv, vv = _view(ks, keep), _view(vs, keep)
    A = _device_A(c, r, q.device)
    rc = N.lib().fc_prefill_attention(
        q.data_ptr(), N.dtype_code(q.dtype), q.stride(0), q.stride(1), q.stride(2), B, Hq, Hkv,
        Sq, D, ks.seq_len - Sq, N.dtype_code(ks.dtype), _jpeg_kind(c), r, c.keep_freqs,
        ks.n_blocks, kv, vv,
        ks._n_raw, N.ptr(A), scale, out.data_ptr(), out.stride(0), out.stride(1), out.stride(2),
        N.stream_ptr(q.device))
    N.check(rc, "fc_prefill_attention")
    return out


def _step_args(ks, vs, query, tokens):
    """The fc_step_args of a (key, value) stream pair with the fields that do
    not change between decode steps filled in (cached on the key stream)."""
    plan = getattr(ks, "_step_plan", None)
    B, Hq, _, D = query.shape
    Hkv = tokens.shape[1]
    dev = query.device
    key = (id(vs), B, Hq, Hkv, D, query.dtype, ks.dtype, dev)
    if plan is not None and plan[0] == key:
        return plan[1], plan[2]
    c = ks.codec
    r = c.block_size
    a = N.StepArgs()
    a.q_dtype = N.dtype_code(query.dtype)
    a.B, a.Hq, a.Hkv, a.D = B, Hq, Hkv, D
    a.store_kind, a.s = _store_kind(c)
    if c.name == "jpeg":
        a.quant_bits = c.quant_bits
        a.basis = dct_basis_device(r, c.keep_freqs, dev).data_ptr()
    else:
        a.keep_m = c.keep_m
    a.stream_dtype = N.dtype_code(ks.dtype)
    a.r = r
    a.A = _device_A(c, r, dev).data_ptr()
    a.n_cu = N.num_cus(dev)
    L = N.lib()
    most = L.fc_attention_splits(a.store_kind, a.stream_dtype, a.q_dtype, a.s, 1 << 40, B, Hkv,
                                 Hq // Hkv, D, a.n_cu)
    ws_bytes = L.fc_attention_workspace_bytes(B, Hq, D, most)
    ks._step_plan = (key, a, ws_bytes)
    return a, ws_bytes


def _same_codec(a, b):
    """Whether two codec objects archive identically (same kind and
    parameters); the fused step archives both streams with one setting."""
    if a is b:
        return True
    return (a.name == b.name and a.block_size == b.block_size
            and getattr(a, "keep_freqs", None) == getattr(b, "keep_freqs", None)
            and getattr(a, "quant_bits", None) == getattr(b, "quant_bits", None)
            and getattr(a, "quant_group", None) == getattr(b, "quant_group", None)
            and getattr(a, "keep_ratio", None) == getattr(b, "keep_ratio", None)
            and getattr(a, "packed", None) == getattr(b, "packed", None))


def codec_decode_step(query, key_tokens, value_tokens, key_stream, value_stream, scale=None):
    """One decode step of a layer in one library call: appends the step's
    key and value tokens (B, Hkv, 1, D) to their streams and attends the
    query (B, Hq, 1, D) over the result; the same as
    ``key_stream.append(key_tokens); value_stream.append(value_tokens);
    codec_decode_attention(query, key_stream, value_stream, scale)``
    (flashcodec/patch_attention.py:95-98), which it falls back to when the
    streams are not yet initialised or the shapes do not allow the fused
    call."""
    ks, vs = key_stream, value_stream
    B, Hq, Sq, D = query.shape
    dev_state = getattr(ks, "_dev_state", None)
    if dev_state is not None:
        return _decode_step_device_state(query, key_tokens, value_tokens, ks, vs, scale,
                                         dev_state)
    fused = (Sq == 1 and key_tokens.shape[-2] == 1 and value_tokens.shape[-2] == 1
             and ks.meta is not None and vs.meta is not None and _same_codec(ks.codec, vs.codec)
             and key_tokens.dtype == ks.dtype and value_tokens.dtype == vs.dtype
             and ks.dtype == vs.dtype and ks.n_blocks == vs.n_blocks
             and ks._n_raw == vs._n_raw and key_tokens.shape == value_tokens.shape
             and key_tokens.shape[0] == B and ks.meta[:3] == vs.meta[:3]
             and ks.meta[0] == B and ks.meta[1] == key_tokens.shape[1]
             and query.is_cuda and key_tokens.is_cuda and value_tokens.is_cuda
             and query.stride(-1) == 1 and key_tokens.stride(-1) == 1
             and value_tokens.stride(-1) == 1 and Hq % key_tokens.shape[1] == 0)
    if not fused:
        ks.append(key_tokens)
        vs.append(value_tokens)
        return codec_decode_attention(query, ks, vs, scale=scale)
    r = ks.codec.block_size
    t, nb = ks._n_raw, ks.n_blocks
    for st, tok in ((ks, key_tokens), (vs, value_tokens)):
        st._tail_buffer(tok)
        if st._capacity == 0 or (t + 1 == r and nb + 1 > st._capacity):
            st._grow(nb + 1, tok)
    a, ws_bytes = _step_args(ks, vs, query, key_tokens)
    dev = query.device
    out = torch.empty_like(query)
    a.q, a.q_sb, a.q_sh = query.data_ptr(), query.stride(0), query.stride(1)
    a.n_blocks, a.n_tail = nb, t
    a.scale = D ** -0.5 if scale is None else float(scale)
    a.out, a.o_sb, a.o_sh = out.data_ptr(), out.stride(0), out.stride(1)
    ws = workspace(dev, ws_bytes)
    a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()
    a.stream = N.stream_ptr(dev)
    jpeg = ks.codec.name == "jpeg"
    for sv, st, tok in ((a.key, ks, key_tokens), (a.value, vs, value_tokens)):
        arch = st._archive_tensors()
        sv.rows = arch[0].data_ptr()
        sv.scales = arch[1].data_ptr() if (jpeg and len(arch) > 1) else None
        sv.anchors = None if jpeg else arch[1].data_ptr()
        sv.masks = arch[2].data_ptr() if (not jpeg and len(arch) > 2) else None
        sv.cap = st._capacity
        sv.tail = st._raw_buf.data_ptr()
        sv.token, sv.tok_sb, sv.tok_sh = tok.data_ptr(), tok.stride(0), tok.stride(1)
    N.check(N.lib().fc_decode_step(ctypes.byref(a)), "fc_decode_step")
    if t + 1 == r:
        for st in (ks, vs):
            st.n_blocks += 1
            st.n_archived += r
            st._n_raw = 0
    else:
        ks._n_raw = vs._n_raw = t + 1
    return out


def _decode_step_device_state(query, key_tokens, value_tokens, ks, vs, scale, state):
    """codec_decode_step with the stream counters on the device (graph
    decoding): the enqueued work reads and advances `state` = (n_blocks,
    n_tail) there and is the same at every step; the host counters are
    advanced by the caller once the work has run (graph.advance_host)."""
    if query.shape[-2] != 1 or key_tokens.shape[-2] != 1 or value_tokens.shape[-2] != 1:
        raise ValueError("device-state decode steps take one token per sequence")
    a, ws_bytes = _step_args(ks, vs, query, key_tokens)
    dev = query.device
    out = torch.empty_like(query)
    a.q, a.q_sb, a.q_sh = query.data_ptr(), query.stride(0), query.stride(1)
    a.n_blocks, a.n_tail = max(1, ks.n_blocks), ks._n_raw
    a.scale = query.shape[-1] ** -0.5 if scale is None else float(scale)
    a.out, a.o_sb, a.o_sh = out.data_ptr(), out.stride(0), out.stride(1)
    key = (dev.index, N.stream_ptr(dev))
    ws = _WORKSPACES.get(key)
    if (ws is None or ws.numel() < ws_bytes) and torch.cuda.is_current_stream_capturing():
        raise RuntimeError("run one decode step on the capture stream before capturing: the "
                           "decode-attention workspace must exist (zero-filled) beforehand")
    ws = workspace(dev, ws_bytes)
    a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()
    a.stream = N.stream_ptr(dev)
    jpeg = ks.codec.name == "jpeg"
    for sv, st, tok in ((a.key, ks, key_tokens), (a.value, vs, value_tokens)):
        arch = st._archive_tensors()
        sv.rows = arch[0].data_ptr()
        sv.scales = arch[1].data_ptr() if (jpeg and len(arch) > 1) else None
        sv.anchors = None if jpeg else arch[1].data_ptr()
        sv.masks = arch[2].data_ptr() if (not jpeg and len(arch) > 2) else None
        sv.cap = st._capacity
        sv.tail = st._raw_buf.data_ptr()
        sv.token, sv.tok_sb, sv.tok_sh = tok.data_ptr(), tok.stride(0), tok.stride(1)
    a.state = state.data_ptr()
    try:
        N.check(N.lib().fc_decode_step(ctypes.byref(a)), "fc_decode_step")
    finally:
        a.state = None
    return out
