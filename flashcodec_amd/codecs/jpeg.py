"""JPEG mode: blockwise orthonormal DCT-II along the token axis, keep the k
lowest frequencies, optionally as int8 with one scale per (block,
frequency).

Same functions and semantics as flashcodec/codecs/jpeg.py:24-158; the
arithmetic runs in HIP kernels (libflashcodec_amd.so) on ROCm tensors.
Tensor contract: input (..., S, D), transform axis -2.
"""

import math

import torch

from .. import _native as N

_BASIS_CACHE = {}
_DEVICE_BASIS = {}


def dct_basis(r, k, device=None, dtype=None):
    """Orthonormal DCT-II basis M (k x r): M[j, n] = c_j cos(pi/r (n + 1/2) j),
    c_0 = sqrt(1/r), c_j = sqrt(2/r) (flashcodec/codecs/jpeg.py:24-40).

    Evaluated once per (r, k) in fp32 on the host with the same tensor
    operations as the reference, so the table carries the reference's bits
    (its cos is not correctly rounded, and the archive codes depend on these
    bits).  Rows do not depend on k."""
    key = (int(r), int(k))
    m = _BASIS_CACHE.get(key)
    if m is None:
        n = torch.arange(r, dtype=torch.float32)
        j = torch.arange(k, dtype=torch.float32)
        c = torch.where(j == 0, math.sqrt(1.0 / r), math.sqrt(2.0 / r))
        angle = math.pi / r * (n[None, :] + 0.5) * j[:, None]
        m = c[:, None] * torch.cos(angle)
        _BASIS_CACHE[key] = m
    if device is not None or dtype is not None:
        m = m.to(device=device, dtype=dtype or m.dtype)
    return m


def device_basis(r, k, device):
    """The k x r fp32 basis resident on `device` (uploaded once)."""
    device = torch.device(device)
    key = (int(r), int(k), device.type, device.index)
    m = _DEVICE_BASIS.get(key)
    if m is None:
        m = dct_basis(r, k).to(device).contiguous()
        _DEVICE_BASIS[key] = m
    return m


def _as_rows(x):
    """(..., S, D) -> (rows, S, D) view with unit feature stride."""
    S, D = x.shape[-2], x.shape[-1]
    x3 = x.reshape(-1, S, D)
    if x3.stride(-1) != 1:
        x3 = x3.contiguous()
    return x3


def encode_into(x3, r, k, quant_bits, coeffs, scales, cap, n0, m, s_valid, H=1, group=0):
    """Run the jpeg archive kernel: m blocks of every sequence of x3
    (B, H, S, D) or (BH, S, D) into the store at block offset n0."""
    if x3.dim() == 3:
        B, Hh = x3.shape[0], 1
        sb, sh, ss = x3.stride(0), 0, x3.stride(1)
    else:
        B, Hh = x3.shape[0], x3.shape[1]
        sb, sh, ss = x3.stride(0), x3.stride(1), x3.stride(2)
    D = x3.shape[-1]
    basis = device_basis(r, k, x3.device)
    if group:
        rc = N.lib().fc_jpeg_encode_grouped(
            x3.data_ptr(), N.dtype_code(x3.dtype), B, Hh, sb, sh, ss, s_valid, m, D, r, k,
            basis.data_ptr(), coeffs.data_ptr(), scales.data_ptr(), cap, n0, group,
            N.stream_ptr(x3.device))
        N.check(rc, "fc_jpeg_encode_grouped")
        return
    rc = N.lib().fc_jpeg_encode(
        x3.data_ptr(), N.dtype_code(x3.dtype), B, Hh, sb, sh, ss, s_valid, m, D, r, k,
        basis.data_ptr(), coeffs.data_ptr(), N.ptr(scales), cap, n0, quant_bits,
        N.stream_ptr(x3.device))
    N.check(rc, "fc_jpeg_encode")


def decode_into(store, scales, B, H, cap, a, nblk, D, r, k, out, out_len, token0=0, group=0):
    """Run the jpeg reconstruction kernel for blocks [a, a+nblk) into `out`
    (B, H, T, D) whose row 0 holds token `token0` (token t = block*r + row;
    tokens >= out_len skipped).  The kernel addresses token t at
    base + t * row stride, so the base handed over sits token0 rows before
    `out`; only rows of `out` itself are written."""
    basis = device_basis(r, k, store.device)
    base = out.data_ptr() - token0 * out.stride(2) * out.element_size()
    if group:
        rc = N.lib().fc_jpeg_decode_grouped(
            store.data_ptr(), scales.data_ptr(), B, H, cap, a, nblk, D, r, k, group,
            basis.data_ptr(), base, N.dtype_code(out.dtype), out.stride(0), out.stride(1),
            out.stride(2), out_len, N.stream_ptr(store.device))
        N.check(rc, "fc_jpeg_decode_grouped")
        return
    rc = N.lib().fc_jpeg_decode(
        store.data_ptr(), N.dtype_code(store.dtype), N.ptr(scales), B, H, cap, a, nblk, D, r,
        k, basis.data_ptr(), base, N.dtype_code(out.dtype), out.stride(0),
        out.stride(1), out.stride(2), out_len, N.stream_ptr(store.device))
    N.check(rc, "fc_jpeg_decode")


class _Compress(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, r, k):
        ctx.r, ctx.k, ctx.S, ctx.shape, ctx.dtype = r, k, x.shape[-2], x.shape, x.dtype
        return _compress(x, r, k)

    @staticmethod
    def backward(ctx, g):
        # d coef / d x is the synthesis (transpose) transform, trimmed to S
        gx = _decompress(g.contiguous(), ctx.r, ctx.S)
        return gx.to(ctx.dtype).reshape(ctx.shape), None, None


class _Decompress(torch.autograd.Function):
    @staticmethod
    def forward(ctx, coeffs, r, out_len):
        ctx.r, ctx.n, ctx.k, ctx.dtype = r, coeffs.shape[-3], coeffs.shape[-2], coeffs.dtype
        ctx.out_len = out_len
        return _decompress(coeffs, r, out_len)

    @staticmethod
    def backward(ctx, g):
        # d rec / d coef is the analysis transform of the (zero padded) grad
        gc = _compress(g.contiguous(), ctx.r, ctx.k)
        return gc.to(ctx.dtype), None, None


def _compress(x, r, k):
    N.require_gpu(x)
    lead, S, D = x.shape[:-2], x.shape[-2], x.shape[-1]
    n = (S + r - 1) // r
    x3 = _as_rows(x)
    out = torch.empty((x3.shape[0], n, k, D), dtype=x.dtype, device=x.device)
    if out.numel():
        encode_into(x3, r, k, 0, out, None, n, 0, n, S)
    return out.reshape(*lead, n, k, D)


def _decompress(coeffs, r, out_len=None):
    N.require_gpu(coeffs)
    lead, (n, k, D) = coeffs.shape[:-3], coeffs.shape[-3:]
    # out_len trims the padding; it never extends past the n*r decoded tokens
    T = n * r if out_len is None else max(0, min(int(out_len), n * r))
    c4 = coeffs.reshape(-1, 1, n, k, D) if coeffs.dim() >= 3 else coeffs
    c4 = c4.contiguous()
    BH = c4.shape[0]
    out = torch.empty((BH, 1, T, D), dtype=torch.float32, device=coeffs.device)
    if out.numel():
        decode_into(c4, None, BH, 1, n, 0, n, D, r, k, out, T)
    return out.reshape(*lead, T, D)


def dct_compress(x, r, k):
    """Blockwise DCT projection (..., S, D) -> (..., n_blocks, k, D) in x's
    dtype; the token axis is zero padded to a multiple of r
    (flashcodec/codecs/jpeg.py:55-67).  Differentiable."""
    if torch.is_grad_enabled() and x.requires_grad:
        return _Compress.apply(x, r, k)
    return _compress(x, r, k)


def dct_decompress(coeffs, r, out_len=None):
    """Blockwise reconstruction (..., n, k, D) -> fp32 (..., n*r, D), trimmed
    to out_len tokens when given (flashcodec/codecs/jpeg.py:70-82).
    Differentiable."""
    if torch.is_grad_enabled() and coeffs.requires_grad:
        return _Decompress.apply(coeffs, r, out_len)
    return _decompress(coeffs, r, out_len)


def _row_view(t, width):
    """(..., D) -> (rows, width) view of a contiguous tensor, D a multiple of width."""
    D = t.shape[-1]
    if D % width:
        raise ValueError(f"the feature width {D} is not a multiple of the quantizer group {width}")
    return t.contiguous().reshape(-1, width)


def quantize_coeffs(coeffs, bits=8, group=0):
    """Symmetric int8 quantisation, one scale per (block, frequency) row:
    (..., n, k, D) -> (int8 codes, fp32 scales (..., n, k, 1))
    (flashcodec/codecs/jpeg.py:85-100).  group=32 (this build's extension):
    one scale per 32 features of each row, scales (..., n, k, D/32) — the
    same rule applied to every 32-feature run."""
    if bits != 8:
        raise ValueError(f"only 8-bit coefficient quantization is supported, got bits={bits}")
    if group not in (0, 32):
        raise ValueError(f"quantizer group must be 0 (one scale per row) or 32, got {group}")
    N.require_gpu(coeffs)
    D = coeffs.shape[-1]
    width = group or D
    rows = coeffs.reshape(-1, D) if not group else _row_view(coeffs, width)
    if rows.stride(-1) != 1:
        rows = rows.contiguous()
    codes = torch.empty(coeffs.shape, dtype=torch.int8, device=coeffs.device)
    scales = torch.empty(coeffs.shape[:-1] + (D // width,), dtype=torch.float32,
                         device=coeffs.device)
    if rows.shape[0]:
        rc = N.lib().fc_quantize_rows(rows.data_ptr(), N.dtype_code(rows.dtype), rows.shape[0],
                                      rows.stride(0), width, codes.data_ptr(), scales.data_ptr(),
                                      N.stream_ptr(coeffs.device))
        N.check(rc, "fc_quantize_rows")
    return codes, scales


def dequantize_coeffs(q, scale, dtype=torch.float32):
    """int8 codes + scales -> q.to(dtype) * scale.to(dtype)
    (flashcodec/codecs/jpeg.py:103-105); scales (..., 1) per row or
    (..., D/32) per 32 features (quantize_coeffs with group=32)."""
    N.require_gpu(q, scale)
    D = q.shape[-1]
    groups = scale.shape[-1] if scale.dim() == q.dim() else 1
    width = D // groups if groups else D
    qc = q.contiguous()
    sc = scale.reshape(q.shape[:-1] + (groups,)).to(torch.float32).contiguous()
    out = torch.empty(q.shape, dtype=dtype, device=q.device)
    n_rows = qc.numel() // width if width else 0
    if n_rows:
        rc = N.lib().fc_dequantize_rows(qc.data_ptr(), sc.data_ptr(), n_rows, width,
                                        out.data_ptr(), N.dtype_code(dtype),
                                        N.stream_ptr(q.device))
        N.check(rc, "fc_dequantize_rows")
    return out


class JPEGCodec:
    """JPEG-style lossy frequency-domain codec (stateless, shareable).
    ``quant_bits=8`` stores the kept coefficients as int8 with one fp32 scale
    per (block, frequency) (flashcodec/codecs/jpeg.py:108-158);
    ``quant_group=32`` (this build's extension) gives every 32 features of a
    row their own scale (the per-32 absmax quantizer of flashcodec
    README.md:487-494)."""

    name = "jpeg"

    def __init__(self, block_size=8, keep_freqs=2, quant_bits=0, quant_group=0):
        assert 1 <= keep_freqs <= block_size, f"keep_freqs must be within [1, {block_size}]"
        assert quant_bits in (0, 8), \
            f"quant_bits must be 0 (store in input dtype) or 8, got {quant_bits}"
        assert quant_group in (0, 32) and (quant_group == 0 or quant_bits == 8), \
            f"quant_group must be 0 or 32 (with quant_bits=8), got {quant_group}"
        self.block_size = block_size
        self.keep_freqs = keep_freqs
        self.quant_bits = quant_bits
        self.quant_group = quant_group

    @property
    def quantized(self):
        return self.quant_bits > 0

    def compress(self, x):
        return dct_compress(x, self.block_size, self.keep_freqs)

    def quantize(self, coeffs):
        """Coefficients -> (int8, scale) when quantized, else (None, None)."""
        if not self.quantized:
            return None, None
        return quantize_coeffs(coeffs, self.quant_bits, self.quant_group)

    def decompress(self, coeffs, out_len=None, scales=None):
        if self.quantized:
            assert scales is not None, "quantized codec needs the scales"
            coeffs = dequantize_coeffs(coeffs, scales)
        return dct_decompress(coeffs, self.block_size, out_len)

    def storage_ratio(self):
        """Archive / original elements assuming fp32 input, raw tail excluded:
        k/r, and a further 4x for int8 codes (scales ignored)."""
        ratio = self.keep_freqs / self.block_size
        return ratio / 4.0 if self.quantized else ratio

    def __repr__(self):
        q = f", quant_bits={self.quant_bits}" if self.quantized else ""
        if self.quant_group:
            q += f", quant_group={self.quant_group}"
        return f"JPEGCodec(block_size={self.block_size}, keep_freqs={self.keep_freqs}{q})"
