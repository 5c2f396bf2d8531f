"""PNG mode: per block an anchor (token 0, stream dtype) and r-1 first-order
fp32 deltas, optionally pruned to the Top-M |delta| per (block, feature);
with packed=True only the surviving deltas are stored (fixed rate: keep_m
values and one mask word per (block, feature)).

Same functions and semantics as flashcodec/codecs/png.py:24-107; the
arithmetic runs in HIP kernels (libflashcodec_amd.so) on ROCm tensors.
Tensor contract: input (..., S, D), transform axis -2.
"""

import math

import torch

from .. import _native as N


def keep_count(block_size, keep_ratio):
    """Deltas kept per (block, feature): max(1, ceil((r-1) * keep_ratio)) when
    keep_ratio < 1, 0 (= no pruning) otherwise (png.py:49-55)."""
    assert 0 < keep_ratio <= 1.0, "keep_ratio must be within (0, 1]"
    if keep_ratio >= 1.0:
        return 0
    return max(1, math.ceil((block_size - 1) * keep_ratio))


def encode_into(x, r, keep_m, deltas, anchors, cap, n0, m, s_valid):
    """Run the png archive kernel: m blocks of every sequence of x (B, H, S,
    D) or (BH, S, D) into deltas (BH, cap, r-1, D) / anchors (BH, cap, D)."""
    if x.dim() == 3:
        B, H = x.shape[0], 1
        sb, sh, ss = x.stride(0), 0, x.stride(1)
    else:
        B, H = x.shape[0], x.shape[1]
        sb, sh, ss = x.stride(0), x.stride(1), x.stride(2)
    rc = N.lib().fc_png_encode(
        x.data_ptr(), N.dtype_code(x.dtype), B, H, sb, sh, ss, s_valid, m, x.shape[-1], r,
        keep_m, deltas.data_ptr(), anchors.data_ptr(), cap, n0, N.stream_ptr(x.device))
    N.check(rc, "fc_png_encode")


def encode_packed_into(x, r, keep_m, vals, masks, anchors, cap, n0, m, s_valid):
    """Run the packed png archive kernel: m blocks of every sequence of x
    into vals (BH, cap, keep_m, D) fp32 / masks (BH, cap, D) int32 / anchors
    (BH, cap, D)."""
    if x.dim() == 3:
        B, H = x.shape[0], 1
        sb, sh, ss = x.stride(0), 0, x.stride(1)
    else:
        B, H = x.shape[0], x.shape[1]
        sb, sh, ss = x.stride(0), x.stride(1), x.stride(2)
    rc = N.lib().fc_png_encode_packed(
        x.data_ptr(), N.dtype_code(x.dtype), B, H, sb, sh, ss, s_valid, m, x.shape[-1], r,
        keep_m, vals.data_ptr(), masks.data_ptr(), anchors.data_ptr(), cap, n0,
        N.stream_ptr(x.device))
    N.check(rc, "fc_png_encode_packed")


def decode_packed_into(vals, masks, anchors, B, H, cap, a, nblk, D, r, keep_m, out, out_len,
                       token0=0):
    """Reconstruct blocks [a, a+nblk) of a packed archive into `out` (as
    decode_into)."""
    base = out.data_ptr() - token0 * out.stride(2) * out.element_size()
    rc = N.lib().fc_png_decode_packed(
        vals.data_ptr(), masks.data_ptr(), anchors.data_ptr(), N.dtype_code(anchors.dtype), B, H,
        cap, a, nblk, D, r, keep_m, base, out.stride(0), out.stride(1), out.stride(2), out_len,
        N.stream_ptr(vals.device))
    N.check(rc, "fc_png_decode_packed")


def png_pack(x, block_size, keep_ratio):
    """Packed Top-M png archive of x (..., S, D) (this build's fixed-rate
    form of png_filter's output, see PNGCodec(packed=True)): (vals (..., n,
    keep_m, D) fp32, masks (..., n, D) int32, anchor (..., n, D))."""
    keep_m = keep_count(block_size, keep_ratio)
    if not keep_m:
        raise ValueError("packing needs keep_ratio < 1")
    N.require_gpu(x)
    r = block_size
    lead, S, D = x.shape[:-2], x.shape[-2], x.shape[-1]
    n = (S + r - 1) // r
    x3 = x.reshape(-1, S, D)
    if x3.stride(-1) != 1:
        x3 = x3.contiguous()
    BH = x3.shape[0]
    vals = torch.empty((BH, n, keep_m, D), dtype=torch.float32, device=x.device)
    masks = torch.empty((BH, n, D), dtype=torch.int32, device=x.device)
    anchors = torch.empty((BH, n, D), dtype=x.dtype, device=x.device)
    if BH * n * D:
        encode_packed_into(x3, r, keep_m, vals, masks, anchors, n, 0, n, S)
    return (vals.reshape(*lead, n, keep_m, D), masks.reshape(*lead, n, D),
            anchors.reshape(*lead, n, D))


def png_unpack(vals, masks, block_size):
    """Dense deltas (..., n, r-1, D) fp32 of a packed archive: png_filter's
    output bit for bit."""
    N.require_gpu(vals, masks)
    lead, (n, keep_m, D) = vals.shape[:-3], vals.shape[-3:]
    r = block_size
    v = vals.reshape(-1, n, keep_m, D).contiguous()
    mk = masks.reshape(-1, n, D).contiguous()
    BH = v.shape[0]
    out = torch.empty((BH, n, r - 1, D), dtype=torch.float32, device=vals.device)
    if out.numel():
        rc = N.lib().fc_png_unpack(v.data_ptr(), mk.data_ptr(), BH, 1, n, 0, n, D, r, keep_m,
                                   out.data_ptr(), n, N.stream_ptr(vals.device))
        N.check(rc, "fc_png_unpack")
    return out.reshape(*lead, n, r - 1, D)


def decode_into(deltas, anchors, B, H, cap, a, nblk, D, r, out, out_len, token0=0):
    """Run the png reconstruction kernel for blocks [a, a+nblk) into `out`,
    whose row 0 holds token `token0` (as jpeg.decode_into)."""
    base = out.data_ptr() - token0 * out.stride(2) * out.element_size()
    rc = N.lib().fc_png_decode(
        deltas.data_ptr(), anchors.data_ptr(), N.dtype_code(anchors.dtype), B, H, cap, a, nblk,
        D, r, base, out.stride(0), out.stride(1), out.stride(2), out_len,
        N.stream_ptr(deltas.device))
    N.check(rc, "fc_png_decode")


def png_filter(x, block_size, keep_ratio=1.0):
    """Delta filtering (..., S, D) -> (deltas (..., n, r-1, D) fp32,
    anchor (..., n, D) in x's dtype); the token axis is zero padded to a
    multiple of r.  With keep_ratio < 1 only the Top-M |delta| per (block,
    feature) survive, the rest are multiplied by 0 (png.py:36-60)."""
    keep_m = keep_count(block_size, keep_ratio)
    N.require_gpu(x)
    r = block_size
    lead, S, D = x.shape[:-2], x.shape[-2], x.shape[-1]
    n = (S + r - 1) // r
    x3 = x.reshape(-1, S, D)
    if x3.stride(-1) != 1:
        x3 = x3.contiguous()
    BH = x3.shape[0]
    deltas = torch.empty((BH, n, r - 1, D), dtype=torch.float32, device=x.device)
    anchors = torch.empty((BH, n, D), dtype=x.dtype, device=x.device)
    if BH * n * D:
        encode_into(x3, r, keep_m, deltas, anchors, n, 0, n, S)
    return deltas.reshape(*lead, n, r - 1, D), anchors.reshape(*lead, n, D)


def png_reconstruct(deltas, anchor):
    """Causal reconstruction anchor + running sum of deltas, in the anchor
    dtype: (..., n, r-1, D), (..., n, D) -> (..., n*r, D) (png.py:63-74)."""
    N.require_gpu(deltas, anchor)
    lead, (n, rm1, D) = deltas.shape[:-3], deltas.shape[-3:]
    r = rm1 + 1
    d4 = deltas.reshape(-1, 1, n, rm1, D).to(torch.float32).contiguous()
    a4 = anchor.reshape(-1, 1, n, D).contiguous()
    BH = d4.shape[0]
    out = torch.empty((BH, 1, n * r, D), dtype=anchor.dtype, device=anchor.device)
    if out.numel():
        decode_into(d4, a4, BH, 1, n, 0, n, D, r, out, n * r)
    return out.reshape(*lead, n * r, D)


class PNGCodec:
    """PNG-style prediction-filter codec (stateless, shareable)
    (flashcodec/codecs/png.py:77-107)."""

    name = "png"

    def __init__(self, block_size=8, keep_ratio=1.0, packed=False):
        assert 0 < keep_ratio <= 1.0, "keep_ratio must be within (0, 1]"
        self.block_size = block_size
        self.keep_ratio = keep_ratio
        # packed (this build's extension): store only the keep_m surviving
        # deltas of each (block, feature) plus a mask word, a fixed-rate
        # block-addressable layout (the reference leaves Top-M sparsity
        # unpacked, README.md:580-583)
        self.packed = bool(packed)
        if self.packed:
            m = keep_count(block_size, keep_ratio)
            if not (2 <= block_size <= 16) or not 1 <= m <= min(8, block_size - 1):
                raise ValueError("packed png archives need 2 <= block_size <= 16 and "
                                 "keep_ratio < 1 with at most 8 kept deltas per block "
                                 f"(block_size={block_size}, keep_ratio={keep_ratio} keeps "
                                 f"{m or block_size - 1})")

    @property
    def keep_m(self):
        return keep_count(self.block_size, self.keep_ratio)

    def filter(self, x):
        return png_filter(x, self.block_size, self.keep_ratio)

    def reconstruct(self, deltas, anchor):
        return png_reconstruct(deltas, anchor)

    def storage_ratio(self):
        """Storage ratio for fp32 input: dense anchor + r-1 deltas per block
        of r tokens = 1.0 (flashcodec/codecs/png.py:94-104); packed: anchor +
        keep_m deltas + one mask word per feature, (2 + keep_m) / r."""
        if self.packed:
            return (2 + self.keep_m) / self.block_size
        return 1.0

    def __repr__(self):
        extra = ", packed=True" if self.packed else ""
        return f"PNGCodec(block_size={self.block_size}, keep_ratio={self.keep_ratio}{extra})"
