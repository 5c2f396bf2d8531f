"""numpy front end of the C++ oracle — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module, and only as the checker; the flashcodec_amd package never does.

Arrays are numpy.  A stream dtype is one of "f32", "f16", "bf16"; values of
such streams are passed around as float32 arrays holding exactly
representable values (`values_of` / `encode_as` convert from/to the storage
form: float32, float16, or uint16 bit patterns for bf16).

Parity status (each function's pinning is listed in tests/test_oracle.py):
  jpeg_encode / quantize / jpeg_decode / dequantize / png_encode /
  png_decode: pinned bit-exactly against the golden vectors written from the
  reference (tests/golden/) plus closed-form checks.
  jpeg_encode_grouped / grouped_coefficients (the per-32 absmax archive,
  which the reference has no code for): the pinned quantize applied per
  group; pinned by the one-group case equalling the row quantizer bit for
  bit, per-group absmax-to-127 and half-step error bounds, and the k = r
  round trip bound.
  png_pack / png_unpack (the packed Top-M png archive, which the reference
  leaves unbuilt): pinned by unpack(pack(d)) == d bit for bit on the golden
  png_filter outputs and on planted +-0 / tie columns, by exhaustive small
  columns, and by planted mistakes (a dropped sign word, a shifted rank)
  that those checks catch.
  attention: fp64 by definition (synthesise every block, softmax over all
  tokens), pinned against brute-force dense attention on tiny inputs and the
  reference's torch-path outputs within tolerance.
"""

import ctypes
import math
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "fc_oracle.cpp")
LIB = os.path.join(HERE, "liboracle.so")

DTYPES = {"f32": 0, "f16": 1, "bf16": 2}


def build():
    """Compile the oracle (g++, no fast-math, no fused contractions)."""
    cmd = ["g++", "-O2", "-std=c++17", "-ffp-contract=off", "-fno-fast-math", "-fopenmp",
           "-shared", "-fPIC", SRC, "-o", LIB + ".tmp"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{res.stderr}")
    os.replace(LIB + ".tmp", LIB)
    return LIB


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            build()
        _lib = ctypes.CDLL(LIB)
        _lib.orc_round.restype = ctypes.c_float
        _lib.orc_round.argtypes = [ctypes.c_int, ctypes.c_float]
    return _lib


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


# ---------------------------------------------------------------- dtypes

def values_of(arr, dtype):
    """Storage array -> float32 values."""
    if dtype == "bf16":
        a = np.ascontiguousarray(arr, dtype=np.uint16)
        return (a.astype(np.uint32) << 16).view(np.float32)
    return np.asarray(arr).astype(np.float32)


def encode_as(values, dtype):
    """float32 values (already representable) -> storage array."""
    v = _f32(values)
    if dtype == "f16":
        return v.astype(np.float16)
    if dtype == "bf16":
        return (v.view(np.uint32) >> 16).astype(np.uint16)
    return v


def round_to(values, dtype):
    """Round float32 values to `dtype` (round to nearest even), as float32."""
    v = _f32(values)
    if dtype == "f32":
        return v.copy()
    if dtype == "f16":
        return v.astype(np.float16).astype(np.float32)
    u = v.view(np.uint32).astype(np.uint64)
    lsb = (u >> 16) & 1
    r = ((u + 0x7FFF + lsb) & 0xFFFF0000).astype(np.uint32).view(np.float32)
    return np.where(np.isnan(v), v, r).astype(np.float32)


def round_scalar_c(dtype, f):
    """The C oracle's own rounding of one value (for cross-checks)."""
    return lib().orc_round(DTYPES[dtype], float(f))


# ---------------------------------------------------------------- basis

def dct_basis_closed_form(r, k):
    """M[j, n] = c_j cos(pi/r (n + 1/2) j) in float64 (jpeg.py:24-40)."""
    n = np.arange(r, dtype=np.float64)
    j = np.arange(k, dtype=np.float64)[:, None]
    c = np.where(j == 0, math.sqrt(1.0 / r), math.sqrt(2.0 / r))
    return c * np.cos(math.pi / r * (n[None, :] + 0.5) * j)


def dct_basis_fp32_angle(r, k):
    """The reference's fp32 evaluation order (jpeg.py:32-35) with a correctly
    rounded cos: angle = f32(f32(f32(pi/r) * f32(n + 0.5)) * j), then
    f32(c_j) * f32(cos(angle)).  Differs from torch's table only through
    torch's cos rounding."""
    n = np.arange(r, dtype=np.float32)
    j = np.arange(k, dtype=np.float32)[:, None]
    angle = (np.float32(math.pi / r) * (n[None, :] + np.float32(0.5))) * j
    c = np.where(j == 0, np.float32(math.sqrt(1.0 / r)), np.float32(math.sqrt(2.0 / r)))
    cos = np.cos(angle.astype(np.float64)).astype(np.float32)
    return (c.astype(np.float32) * cos).astype(np.float32)


# ---------------------------------------------------------------- blocks

def to_blocks(x, r):
    """(..., S, D) -> ((n_items, r, D) zero padded, lead shape, n_blocks)."""
    x = _f32(x)
    lead, S, D = x.shape[:-2], x.shape[-2], x.shape[-1]
    n = (S + r - 1) // r
    pad = n * r - S
    if pad:
        x = np.concatenate([x, np.zeros(lead + (pad, D), np.float32)], axis=-2)
    return np.ascontiguousarray(x.reshape(-1, r, D)), lead, n


def jpeg_encode(x, r, k, basis, dtype="f32", quant=False):
    """dct_compress (+ quantize_coeffs).  x: (..., S, D) values of dtype.
    Returns coef (..., n, k, D) [, codes, scales (..., n, k)]."""
    xb, lead, n = to_blocks(x, r)
    items, D = xb.shape[0], xb.shape[-1]
    coef = np.empty((items, k, D), np.float32)
    codes = np.empty((items, k, D), np.int8) if quant else np.empty(1, np.int8)
    scales = np.empty((items, k), np.float32) if quant else np.empty(1, np.float32)
    lib().orc_jpeg_encode(_p(xb), ctypes.c_long(items), r, k, ctypes.c_long(D),
                          _p(_f32(basis)), DTYPES[dtype], int(quant), _p(coef), _p(codes),
                          _p(scales))
    coef = coef.reshape(lead + (n, k, D))
    if not quant:
        return coef
    return coef, codes.reshape(lead + (n, k, D)), scales.reshape(lead + (n, k))


def quantize(c, dtype="f32"):
    """quantize_coeffs over the last axis: (..., D) -> codes, scales (...)."""
    c = _f32(c)
    D = c.shape[-1]
    rows = c.reshape(-1, D)
    codes = np.empty(rows.shape, np.int8)
    scales = np.empty(rows.shape[0], np.float32)
    lib().orc_quantize(_p(rows), ctypes.c_long(rows.shape[0]), ctypes.c_long(D),
                       DTYPES[dtype], _p(codes), _p(scales))
    return codes.reshape(c.shape), scales.reshape(c.shape[:-1])


def jpeg_encode_grouped(x, r, k, basis, dtype="f32", group=32):
    """dct_compress, then the quantize_coeffs rule applied to every `group`
    features of a coefficient row (each run gets its own absmax scale: the
    per-32 absmax quantizer of flashcodec README.md:487-494, which the
    reference describes but does not ship).  Returns coef (..., n, k, D),
    codes (..., n, k, D), scales (..., n, k, D/group)."""
    coef = jpeg_encode(x, r, k, basis, dtype)
    D = coef.shape[-1]
    assert D % group == 0, "D must be a multiple of the group"
    codes, scales = quantize(coef.reshape(coef.shape[:-1] + (D // group, group)), dtype)
    return coef, codes.reshape(coef.shape), scales


def grouped_coefficients(codes, scales):
    """fp32 codes * scale of each feature's group: (..., D) codes with
    (..., D/g) scales -> (..., D) (the fp32 products the decode takes)."""
    codes = np.asarray(codes, np.int8)
    g = codes.shape[-1] // scales.shape[-1]
    return codes.astype(np.float32) * np.repeat(_f32(scales), g, axis=-1)


def dequantize(codes, scales, dtype="f32"):
    codes = np.ascontiguousarray(codes, np.int8)
    D = codes.shape[-1]
    out = np.empty(codes.shape, np.float32)
    lib().orc_dequantize(_p(codes), _p(_f32(scales)), ctypes.c_long(codes.size // D),
                         ctypes.c_long(D), DTYPES[dtype], _p(out))
    return out


def jpeg_decode(coef, r, basis, out_dtype="f32", codes=None, scales=None):
    """dct_decompress (of dequantised codes when `codes` is given).
    coef/codes: (..., n, k, D) -> (..., n*r, D) values of out_dtype."""
    src = codes if codes is not None else coef
    lead, (n, k, D) = src.shape[:-3], src.shape[-3:]
    items = int(np.prod(lead, dtype=np.int64)) * n
    out = np.empty((items, r, D), np.float32)
    quant = codes is not None
    cf = np.empty(1, np.float32) if quant else _f32(coef).reshape(items, k, D)
    cd = np.ascontiguousarray(codes, np.int8).reshape(items, k, D) if quant else np.empty(1, np.int8)
    sc = _f32(scales).reshape(items, k) if quant else np.empty(1, np.float32)
    lib().orc_jpeg_decode(_p(cf), _p(cd), _p(sc), int(quant), ctypes.c_long(items), r, k,
                          ctypes.c_long(D), _p(_f32(basis)), DTYPES[out_dtype], _p(out))
    return out.reshape(lead + (n * r, D))


def png_keep_m(r, keep_ratio):
    """Steps kept per (block, feature) (png.py:49-55); 0 = no pruning."""
    if keep_ratio >= 1.0:
        return 0
    return max(1, math.ceil((r - 1) * keep_ratio))


def png_encode(x, r, keep_ratio=1.0):
    """png_filter.  Returns deltas (..., n, r-1, D) fp32, anchors (..., n, D)."""
    xb, lead, n = to_blocks(x, r)
    items, D = xb.shape[0], xb.shape[-1]
    deltas = np.empty((items, r - 1, D), np.float32)
    anchors = np.empty((items, D), np.float32)
    lib().orc_png_encode(_p(xb), ctypes.c_long(items), r, ctypes.c_long(D),
                         png_keep_m(r, keep_ratio), _p(deltas), _p(anchors))
    return deltas.reshape(lead + (n, r - 1, D)), anchors.reshape(lead + (n, D))


def topk_keep(values, m):
    """torch CPU topk(m) selection of one column, as a bool keep mask."""
    v = _f32(values)
    keep = np.zeros(v.shape[0], np.uint8)
    lib().orc_topk_keep(_p(v), int(v.shape[0]), int(m), _p(keep))
    return keep.astype(bool)


def png_decode(deltas, anchors, dtype="f32"):
    """png_reconstruct: (..., n, r-1, D), (..., n, D) -> (..., n*r, D)."""
    lead, (n, rm1, D) = deltas.shape[:-3], deltas.shape[-3:]
    r = rm1 + 1
    items = int(np.prod(lead, dtype=np.int64)) * n
    out = np.empty((items, r, D), np.float32)
    lib().orc_png_decode(_p(_f32(deltas).reshape(items, rm1, D)),
                         _p(_f32(anchors).reshape(items, D)), ctypes.c_long(items), r,
                         ctypes.c_long(D), DTYPES[dtype], _p(out))
    return out.reshape(lead + (n * r, D))


# ---------------------------------------------------------------- packed png

PACK_SIGN_SHIFT = 16   # mask word: bits 0..14 kept steps, bits 16..30 pruned-zero signs


def png_pack(deltas, keep_m):
    """Fixed-rate packing of png_filter's Top-M deltas (png.py:36-60: at most
    keep_m of the r-1 steps of a (block, feature) column survive; the others
    are +-0.0, the sign of the pruned delta kept).  This build's archive
    format, which the reference leaves unbuilt (README.md:580-583):
      vals (..., n, keep_m, D) fp32: the column's kept steps in step order;
      mask (..., n, D) uint32: bit i = step i kept; bit 16 + i = sign bit
        of step i when it is not kept (0 for kept steps).
    Kept steps: every step whose bits are not +-0 (at most keep_m of them),
    then the lowest-index +-0 steps until there are keep_m (a kept or a
    pruned zero unpacks to the same bits).  r - 1 <= 15 steps.  Raises when
    a column has more than keep_m non-zero steps (png_filter's pruned
    non-finite deltas become NaN, which the format does not hold)."""
    d = np.ascontiguousarray(deltas, np.float32)
    *lead, n, rm1, D = d.shape
    if not 1 <= keep_m <= rm1 or rm1 > 15:
        raise ValueError(f"packing needs 1 <= keep_m <= r-1 <= 15 (keep_m={keep_m}, r-1={rm1})")
    bits = d.view(np.uint32)
    nz = (bits & 0x7FFFFFFF) != 0                                  # (..., n, rm1, D)
    cnt = nz.sum(axis=-2)
    if (cnt > keep_m).any():
        raise ValueError("a column holds more than keep_m non-zero deltas")
    # fill with the lowest-index zero steps: rank of each zero among zeros
    zero_rank = np.cumsum(~nz, axis=-2) - 1
    need = (keep_m - cnt)[..., None, :]
    kept = nz | (~nz & (zero_rank < need))
    steps = np.arange(rm1, dtype=np.uint32).reshape((rm1, 1))
    kept_bits = (kept.astype(np.uint32) << steps).sum(axis=-2, dtype=np.uint32)
    sign = ((bits >> 31) & 1).astype(np.uint32) * (~kept)
    sign_bits = (sign << (steps + PACK_SIGN_SHIFT)).sum(axis=-2, dtype=np.uint32)
    mask = (kept_bits | sign_bits).astype(np.uint32)
    # slot j of a column = its j-th kept step
    order = np.argsort(~kept, axis=-2, kind="stable")[..., :keep_m, :]
    vals = np.take_along_axis(d, order, axis=-2)
    return vals, mask


def png_unpack(vals, mask, r):
    """Dense deltas (..., n, r-1, D) fp32 of a packed archive: step i is the
    column's next kept value when bit i of its mask word is set, else a zero
    with the sign bit 16 + i (the inverse of png_pack, bit for bit)."""
    v = np.ascontiguousarray(vals, np.float32)
    m = np.ascontiguousarray(mask, np.uint32)
    *lead, n, keep_m, D = v.shape
    rm1 = r - 1
    steps = np.arange(rm1, dtype=np.uint32).reshape((rm1, 1))
    kept = ((m[..., None, :] >> steps) & 1).astype(bool)            # (..., n, rm1, D)
    rank = np.cumsum(kept, axis=-2) - 1
    picked = np.take_along_axis(v, np.clip(rank, 0, keep_m - 1), axis=-2)
    sign = (m[..., None, :] >> (steps + PACK_SIGN_SHIFT)) & 1
    zero = (sign << 31).astype(np.uint32).view(np.float32)
    return np.where(kept, picked, zero).astype(np.float32)


# ---------------------------------------------------------------- attention

def synthesis_matrix(mode, r, basis=None):
    """A (r x s): jpeg M^T (attention.py:35-42), png tril(1)."""
    if mode == "jpeg":
        return np.ascontiguousarray(np.asarray(basis, np.float64).T)
    return np.tril(np.ones((r, r), np.float64))


def attention(q, rows_k, rows_v, raw_k, raw_v, A, scale, n_threads=1):
    """fp64 decode attention by definition.
    q (B, Hq, D); rows (B, Hkv, nb, s, D); raw (B, Hkv, nr, D); -> (B, Hq, D)."""
    q = np.ascontiguousarray(q, np.float64)
    B, Hq, D = q.shape
    Hkv, nb, s = rows_k.shape[1], rows_k.shape[2], rows_k.shape[3]
    r = A.shape[0]
    nr = 0 if raw_k is None else raw_k.shape[2]
    rk = np.ascontiguousarray(rows_k, np.float64)
    rv = np.ascontiguousarray(rows_v, np.float64)
    zk = np.ascontiguousarray(raw_k if raw_k is not None else np.zeros(1), np.float64)
    zv = np.ascontiguousarray(raw_v if raw_v is not None else np.zeros(1), np.float64)
    out = np.empty((B, Hq, D), np.float64)
    L = ctypes.c_long
    lib().orc_attention(_p(q), _p(rk), _p(rv), _p(zk), _p(zv),
                        _p(np.ascontiguousarray(A, np.float64)), L(B), L(Hq), L(Hkv), L(nb),
                        int(r), int(s), L(nr), L(D), ctypes.c_double(scale), _p(out),
                        int(n_threads))
    return out


def stored_rows_jpeg(codes_or_coef, scales=None):
    """Dequantised jpeg rows (fp64) from codes * scales or float coefficients;
    scales (..., k) per row or (..., k, D/g) per g features."""
    if scales is None:
        return np.asarray(codes_or_coef, np.float64)
    if np.ndim(scales) == np.ndim(codes_or_coef):
        return grouped_coefficients(codes_or_coef, scales).astype(np.float64)
    return np.asarray(codes_or_coef, np.float64) * np.asarray(scales, np.float32).astype(
        np.float32)[..., None].astype(np.float64)


def stored_rows_png(deltas, anchors):
    """png rows (anchor, deltas) stacked on the row axis (attention.py:59-61)."""
    return np.concatenate([np.asarray(anchors, np.float64)[..., None, :],
                           np.asarray(deltas, np.float64)], axis=-2)


# ---------------------------------------------------------------- inputs

def ar1(shape, rho, seed, scale=None):
    """AR(1) along axis -2 with unit stationary variance (numpy PCG64):
    x_0 ~ N(0,1), x_t = rho x_{t-1} + sqrt(1-rho^2) eps_t; optional
    per-channel scale (broadcast over the token axis)."""
    rng = np.random.Generator(np.random.PCG64(seed))
    *lead, S, D = shape
    eps = rng.standard_normal(tuple(lead) + (S, D)).astype(np.float32)
    x = np.empty_like(eps)
    x[..., 0, :] = eps[..., 0, :]
    c = np.float32(math.sqrt(1.0 - rho * rho))
    for t in range(1, S):
        x[..., t, :] = np.float32(rho) * x[..., t - 1, :] + c * eps[..., t, :]
    if scale is not None:
        x = x * scale
    return x
