"""torch-CPU restatement of the reference's portable decode attention and
codec operations — TEST INFRASTRUCTURE ONLY.

Only bench.py's cpu_baseline legs (as the timed CPU baselines) and tests/
(which pin it) use this module; the flashcodec_amd package never does.

Codec operations (the CPU baselines of the C1 / C2 / C4 workloads), the
reference's tensor operations in its order, so that on the same torch CPU
build they produce the reference's bits: dct_compress / quantize /
dequantize / dct_decompress (flashcodec/codecs/jpeg.py:43-105), png_filter /
png_reconstruct (flashcodec/codecs/png.py:24-74).

The reference's `codec_decode_attention(..., impl="torch")`
(flashcodec/attention.py:101-140) on stored rows that are already
dequantised, with the same tensor operations in the same order, so that on
the same torch CPU build it produces the reference's own bits:
  * stored rows of the jpeg int8 archive dequantised into the query dtype as
    codes.to(dtype) * scales.to(dtype) (flashcodec/attention.py:45-61,
    flashcodec/codecs/jpeg.py:103-105); png rows are anchor + deltas in fp32;
  * GQA by viewing the query as (B, Hk, G, 1, D);
  * per-block scores against the s stored rows, mapped to the r token logits
    through A (r x s), raw-tail logits appended, softmax in fp32 with the
    scale applied after the cast, probabilities cast back to the work dtype;
  * output weights w = p_block A per stored row, out = w . rows + p_raw . V_raw.

Parity status: pinned in tests/test_oracle.py against the reference's own
torch-path outputs (golden vectors written from the reference, bit-exact on
this container's torch CPU) and against the fp64 oracle within tolerance.
"""

import math

import torch


def _blocks(x, r):
    """Zero-pad the token axis to a multiple of r and view it as (..., n, r,
    D) (flashcodec/codecs/jpeg.py:43-52)."""
    S = x.shape[-2]
    n = (S + r - 1) // r
    if n * r != S:
        x = torch.nn.functional.pad(x, (0, 0, 0, n * r - S))
    return x.reshape(*x.shape[:-2], n, r, x.shape[-1])


def dct_compress(x, r, basis):
    """(..., S, D) -> (..., n, k, D) in x's dtype: fp32 product with the
    k x r basis along each block (flashcodec/codecs/jpeg.py:55-67)."""
    hp = _blocks(x, r).float().transpose(-2, -1)
    return torch.matmul(hp, basis.t()).transpose(-2, -1).to(x.dtype)


def quantize(coeffs):
    """Per-(block, frequency) absmax int8 quantizer: (codes, fp32 scales)
    (flashcodec/codecs/jpeg.py:85-100)."""
    amax = coeffs.abs().amax(dim=-1, keepdim=True)
    scale = amax / 127.0
    scale = torch.where(scale > 0, scale, torch.ones_like(scale))
    q = torch.round(coeffs.float() / scale).clamp_(-127, 127).to(torch.int8)
    return q, scale.to(torch.float32)


def dequantize(q, scale, dtype=torch.float32):
    """codes x scale in `dtype` (flashcodec/codecs/jpeg.py:103-105)."""
    return q.to(dtype) * scale.to(dtype)


def dct_decompress(coeffs, r, basis):
    """(..., n, k, D) -> (..., n * r, D) fp32 (flashcodec/codecs/jpeg.py:70-82)."""
    n = coeffs.shape[-3]
    hp = torch.matmul(coeffs.transpose(-2, -1).float(), basis)
    return hp.transpose(-2, -1).reshape(*coeffs.shape[:-3], n * r, coeffs.shape[-1])


def png_filter(x, r, keep_ratio=1.0):
    """(deltas (..., n, r-1, D) fp32, anchors (..., n, D)): Top-M by |delta|
    per (block, feature) when keep_ratio < 1 (flashcodec/codecs/png.py:36-60)."""
    blocks = _blocks(x, r)
    anchor = blocks[..., 0, :]
    bf = blocks.float()
    delta = bf[..., 1:, :] - bf[..., :-1, :]
    if keep_ratio < 1.0:
        m = max(1, math.ceil(delta.shape[-2] * keep_ratio))
        topi = delta.abs().topk(m, dim=-2).indices
        mask = torch.zeros_like(delta, dtype=torch.bool)
        mask.scatter_(-2, topi, True)
        delta = delta * mask
    return delta, anchor


def png_reconstruct(deltas, anchor):
    """anchor + cumsum of the deltas, in the anchor dtype, (..., n * r, D)
    (flashcodec/codecs/png.py:63-74)."""
    base = anchor.float().unsqueeze(-2)
    rec = torch.cat([base, base + torch.cumsum(deltas.float(), dim=-2)], dim=-2)
    return rec.to(anchor.dtype).reshape(*rec.shape[:-3], rec.shape[-3] * rec.shape[-2],
                                        rec.shape[-1])


def jpeg_rows(codes, scales, dtype):
    """Dequantised jpeg int8 rows in `dtype`: codes (B, H, n, s, D) int8,
    scales (B, H, n, s, 1) fp32 (flashcodec/codecs/jpeg.py:103-105)."""
    return codes.to(dtype) * scales.to(dtype)


def png_rows(deltas, anchors):
    """png stored rows (B, H, n, r, D) fp32: the anchor on row 0, the r-1
    deltas after it (flashcodec/attention.py:58-61)."""
    return torch.cat([anchors.unsqueeze(-2).float(), deltas.float()], dim=-2)


def decode_attention(query, k_rows, v_rows, k_raw, v_raw, A, scale):
    """One decode step of attention over archived rows plus a raw tail.

    query (B, Hq, 1, D); k_rows / v_rows (B, Hk, n, s, D) in the work dtype
    or None (no archived block); k_raw / v_raw (B, Hk, t, D) or None;
    A (r, s) synthesis matrix; scale a float.  Returns (B, Hq, 1, D) in the
    query dtype.  flashcodec/attention.py:101-140.
    """
    B, Hq, _, D = query.shape
    if k_rows is None and k_raw is None:
        return torch.zeros_like(query)
    Hk = (k_rows if k_rows is not None else k_raw).shape[1]
    G = Hq // Hk
    wd = k_rows.dtype if k_rows is not None else torch.float32
    qg = query.to(wd).reshape(B, Hk, G, 1, D)
    parts = []
    out = torch.zeros(B, Hk, G, D, dtype=wd)
    if k_rows is not None:
        Aw = A.to(wd)
        per_row = torch.einsum("bhgqd,bhnsd->bhgns", qg, k_rows)
        parts.append(torch.einsum("bhgns,rs->bhgnr", per_row, Aw).flatten(-2))
    if k_raw is not None:
        parts.append(torch.einsum("bhgqd,bhtd->bhgt", qg, k_raw.to(wd)))
    probs = torch.softmax(torch.cat(parts, dim=-1).float() * scale, dim=-1).to(wd)
    used = 0
    if k_rows is not None:
        n, r = k_rows.shape[2], A.shape[0]
        p_blk = probs[..., :n * r].reshape(B, Hk, G, n, r)
        w = torch.einsum("bhgnr,rs->bhgns", p_blk, Aw)
        out = out + torch.einsum("bhgns,bhnsd->bhgd", w, v_rows)
        used = n * r
    if k_raw is not None:
        out = out + torch.einsum("bhgt,bhtd->bhgd", probs[..., used:], v_raw.to(wd))
    return out.reshape(B, Hq, 1, D).to(query.dtype)
