"""torch-CPU restatement of the reference's portable decode attention —
TEST INFRASTRUCTURE ONLY.

Only bench.py's cpu_baseline leg (as the timed CPU baseline) and tests/
(which pin it) use this module; the flashcodec_amd package never does.

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

import torch


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
