"""Materialisation-free decode attention on the codec archive.

Both codecs are linear along the token axis: an archived block of r tokens
is A @ S with S its s stored rows and A (r x s) the synthesis matrix (jpeg:
the DCT basis transposed; png: tril(1) over anchor + deltas).  For one query
token the scores are (q . S^T) A^T and the output (prob A) S, so the (S, D)
reconstruction never exists (flashcodec/attention.py:1-27).

`codec_decode_attention` keeps the reference signature
(flashcodec/attention.py:64) and runs two HIP kernels of
libflashcodec_amd.so: a split-K pass over the archived blocks (every kv
head's rows read once per group of up to eight query heads) and a merge pass
that folds in the raw tail.
"""

import torch

from . import _native as N
from .codecs import dct_basis

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
    stream = torch.cuda.current_stream(device).cuda_stream
    key = (device.index, stream)
    ws = _WORKSPACES.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = torch.zeros(nbytes, dtype=torch.uint8, device=device)
        _WORKSPACES[key] = ws
    return ws


def _view(stream, keep):
    """fc_stream_view of a stream; tensors it points into are added to `keep`."""
    v = N.StreamView()
    c = stream.codec
    if stream.n_blocks:
        if c.name == "jpeg":
            v.rows = stream._coeffs.data_ptr()
            v.scales = stream._scales.data_ptr() if c.quantized else None
        else:
            v.rows = stream._deltas.data_ptr()
            v.anchors = stream._anchors.data_ptr()
        v.cap = stream._capacity
    if stream.raw is not None:
        raw = stream.raw if stream.raw.stride(-1) == 1 else stream.raw.contiguous()
        keep.append(raw)
        v.raw = raw.data_ptr()
        v.raw_sb, v.raw_sh, v.raw_st = raw.stride(0), raw.stride(1), raw.stride(2)
    return v


def codec_decode_attention(query, key_stream, value_stream, scale=None, impl="auto",
                           _n_splits=None):
    """Attention of one new query token against a codec archive without
    materialising the reconstructed KV.

    Args:
        query: (B, Hq, 1, D) query of the current step.
        key_stream, value_stream: ``_CodecStream`` instances of one layer.
        scale: attention scale (default ``D ** -0.5``).
        impl: ``"auto"`` / ``"hip"`` (``"triton"`` is accepted as the name of
            the reference's accelerated path and runs the same HIP kernels).
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
    if impl not in ("auto", "hip", "triton"):
        raise ValueError(f"impl={impl!r}: this build computes on HIP kernels only "
                         "(use 'auto' or 'hip')")
    scale = D ** -0.5 if scale is None else float(scale)
    ks, vs = key_stream, value_stream
    if ks.codec.name != vs.codec.name:
        raise ValueError("key and value streams must use the same codec")
    nb = ks.n_blocks
    if vs.n_blocks != nb or vs.n_archived != ks.n_archived:
        raise ValueError("key and value streams hold different token counts")
    n_raw = 0 if ks.raw is None else ks.raw.shape[-2]
    if nb == 0 and n_raw == 0:
        return torch.zeros_like(query)                   # empty cache
    N.require_gpu(query)
    like = ks.raw if nb == 0 else ks._archive_tensors()[0]
    N.require_gpu(like)
    Hkv = like.shape[1]
    assert Hq % Hkv == 0, f"query heads ({Hq}) must be a multiple of kv heads ({Hkv})"
    if like.shape[0] != B:
        raise ValueError(f"batch mismatch: query {B}, cache {like.shape[0]}")

    c = ks.codec
    r = ks.block_size
    if c.name == "jpeg":
        kind = N.STORE_JPEG_I8 if c.quantized else N.STORE_JPEG_FP
        s = c.keep_freqs
    else:
        kind = N.STORE_PNG
        s = r
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
