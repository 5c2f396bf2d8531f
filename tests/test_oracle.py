"""CPU: pin the oracle against the reference's golden vectors, the
mathematics, and the library routines the reference runs on.

Pinning map of oracle/oracle.py:
  round_to / orc_round   -> torch's CPU casts (library routine)
  dct basis bits         -> golden basis (reference dct_basis); closed form
                            within 2 ulp; orthonormality
  jpeg_encode (+quant)   -> golden dct_compress / quantize_coeffs bits;
                            k = r lossless; |q| <= 127, error <= scale/2;
                            zero block -> scale 1
  jpeg_decode/dequantize -> golden dct_decompress / dequantize_coeffs bits
  topk_keep              -> torch.topk on tie-heavy columns; golden png
  png_encode/png_decode  -> golden png_filter / png_reconstruct bits;
                            bf16 / f32 keep=1 lossless; kept count == m
  stream (append/read)   -> golden _CodecStream archives, read() and crop
  attention              -> golden torch-path outputs; dense attention on
                            the golden reconstructed view
Pinning map of oracle/torch_path.py (bench.py's CPU baseline):
  decode_attention       -> the reference's impl="torch" outputs (golden),
                            bit-exact; fp64 attention within tolerance; a
                            planted mistake (tail dropped) is caught
"""

import math

import numpy as np
import pytest
import torch

TORCH_DT = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}


def _bits(a):
    a = np.ascontiguousarray(a)
    return a.view(np.uint32) if a.dtype == np.float32 else a


def _torch_values(storage, dtype):
    if dtype == "bf16":
        return torch.from_numpy(storage.view(np.int16).copy()).view(torch.bfloat16).float()
    return torch.from_numpy(np.asarray(storage).copy()).float()


# ---------------------------------------------------------------- rounding

def test_rounding_matches_torch_casts(oracle):
    rng = np.random.default_rng(0)
    v = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * 10 ** rng.uniform(-9, 5, 20000),
        np.float32([0.0, -0.0, 65504, 65519.9, 65520, 1e-8, 6e-8, 5.96e-8, 3e-8, 2.98e-8,
                    1 + 2 ** -11, 1 + 3 * 2 ** -11, 1 + 2 ** -8, 1 + 3 * 2 ** -8, -1e30]),
    ]).astype(np.float32)
    t = torch.from_numpy(v)
    for dt in ("f16", "bf16"):
        ref = t.to(TORCH_DT[dt]).float().numpy()
        with np.errstate(over="ignore"):
            got = oracle.round_to(v, dt)
        assert np.array_equal(_bits(got), _bits(ref)), dt
        sample = v[::97]
        c = np.float32([oracle.round_scalar_c(dt, f) for f in sample])
        assert np.array_equal(_bits(c), _bits(ref[::97])), dt


# ---------------------------------------------------------------- basis

@pytest.mark.parametrize("r", [2, 4, 8, 12, 16, 32, 64])
def test_basis_bits_match_reference(golden, r):
    from flashcodec_amd import dct_basis
    g = golden("basis").data[f"r{r}"]
    mine = dct_basis(r, r).numpy()
    assert np.array_equal(_bits(mine), _bits(g))
    for k in (1, max(1, r // 2), r):
        assert np.array_equal(_bits(dct_basis(r, k).numpy()), _bits(g[:k]))


@pytest.mark.parametrize("r", [2, 4, 8, 12, 16, 32, 64])
def test_basis_closed_form_and_orthonormal(golden, oracle, r):
    g = golden("basis").data[f"r{r}"]
    # same fp32 angle, correctly rounded cos: torch's cos is within an ulp
    f32 = oracle.dct_basis_fp32_angle(r, r)
    ulp = np.spacing(np.abs(f32)).astype(np.float64)
    assert np.all(np.abs(g.astype(np.float64) - f32) <= 2 * ulp)
    # and the table is the orthonormal DCT-II up to the fp32 angle error
    # (which grows with r: the angle reaches ~pi * r)
    exact = oracle.dct_basis_closed_form(r, r)
    assert np.abs(g - exact).max() < 1e-7 * r
    assert np.allclose(g.astype(np.float64) @ g.T, np.eye(r), atol=max(1e-6, 2e-7 * r))


# ---------------------------------------------------------------- jpeg

def _jpeg_cases():
    from tests.conftest import Golden
    return Golden("jpeg").names()


@pytest.mark.parametrize("name", _jpeg_cases())
def test_jpeg_oracle_matches_reference(golden, oracle, name):
    G = golden("jpeg")
    c, m = G.case(name), G.meta[name]
    dt, r, k = m["dtype"], m["r"], m["k"]
    basis = golden("basis").data[f"r{r}"][:k]
    x = oracle.values_of(c["x"], dt)
    coef, codes, scales = oracle.jpeg_encode(x, r, k, basis, dt, quant=True)
    assert np.array_equal(_bits(coef), _bits(oracle.values_of(c["coef"], dt)))
    assert np.array_equal(codes, c["codes"])
    assert np.array_equal(_bits(scales), _bits(c["scales"]))
    deq = oracle.dequantize(codes, scales, "f32")
    assert np.array_equal(_bits(deq), _bits(c["deq_f32"]))
    deq_t = oracle.dequantize(codes, scales, dt)
    assert np.array_equal(_bits(deq_t), _bits(oracle.values_of(c["deq_T"], dt)))
    S = m["shape"][-2]
    rec = oracle.jpeg_decode(coef, r, basis, "f32")[..., :S, :]
    assert np.array_equal(_bits(rec), _bits(c["rec"]))
    rec_q = oracle.jpeg_decode(None, r, basis, "f32", codes=codes, scales=scales)[..., :S, :]
    assert np.array_equal(_bits(rec_q), _bits(c["rec_q"]))


@pytest.mark.parametrize("name", _jpeg_cases())
def test_torch_path_codec_matches_reference(golden, name):
    """oracle/torch_path.py's jpeg operations (bench.py's C1 / C2 CPU
    baselines) reproduce the reference's bits on this torch CPU build."""
    from oracle import torch_path as T
    G = golden("jpeg")
    c, m = G.case(name), G.meta[name]
    dt, r, k = m["dtype"], m["r"], m["k"]
    basis = torch.from_numpy(np.ascontiguousarray(golden("basis").data[f"r{r}"][:k]))
    x = _torch_of(c["x"], dt)
    coef = T.dct_compress(x, r, basis)
    assert np.array_equal(_bits(_np_of(coef, dt)), _bits(c["coef"]))
    codes, scales = T.quantize(coef)
    assert np.array_equal(codes.numpy(), c["codes"])
    assert np.array_equal(_bits(scales[..., 0].numpy()), _bits(c["scales"]))
    S = m["shape"][-2]
    rec_q = T.dct_decompress(T.dequantize(codes, scales), r, basis)[..., :S, :]
    assert np.array_equal(_bits(rec_q.numpy()), _bits(c["rec_q"]))


def _torch_of(storage, dt):
    a = np.ascontiguousarray(storage)
    if dt == "bf16":
        return torch.from_numpy(a.view(np.int16).copy()).view(torch.bfloat16)
    return torch.from_numpy(a.copy())


def _np_of(t, dt):
    if dt == "bf16":
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def test_jpeg_closed_form_properties(golden, oracle):
    rng = np.random.default_rng(3)
    r = 8
    basis = golden("basis").data["r8"]
    x = rng.standard_normal((2, 3, 64, 32)).astype(np.float32)
    # k == r is an orthonormal change of basis: lossless up to fp32 rounding
    rec = oracle.jpeg_decode(oracle.jpeg_encode(x, r, r, basis, "f32"), r, basis, "f32")
    assert np.abs(rec - x).max() < 1e-5
    # quantiser bounds
    coef, codes, scales = oracle.jpeg_encode(x, r, 2, basis[:2], "f32", quant=True)
    assert np.abs(codes.astype(np.int32)).max() <= 127
    err = np.abs(codes * scales[..., None] - coef)
    assert np.all(err <= scales[..., None] / 2 * (1 + 1e-6))
    # the largest |coefficient| of a row maps to +-127
    assert np.all(np.abs(codes).max(-1) == 127)
    # all-zero block: scale 1, codes 0
    z = np.zeros((1, 1, 8, 16), np.float32)
    _, zc, zs = oracle.jpeg_encode(z, r, 4, basis[:4], "f16", quant=True)
    assert np.all(zs == 1.0) and np.all(zc == 0)
    # a planted mistake (reversed tap order) is caught by the golden bits
    G = golden("jpeg")
    c, m = G.case("f32_r8k2"), G.meta["f32_r8k2"]
    xg = oracle.values_of(c["x"], "f32")
    flipped = oracle.jpeg_encode(xg[..., ::-1, :].copy(), 8, 2, basis[:2, ::-1].copy(), "f32")
    assert not np.array_equal(_bits(flipped), _bits(c["coef"]))


def _group_bounds_hold(coef, codes, scales, g):
    """Per-group quantizer invariants: codes within +-127, every group with
    a nonzero absmax reaches +-127, |code * s - c| <= s / 2."""
    cg = coef.reshape(coef.shape[:-1] + (-1, g))
    qg = codes.reshape(cg.shape).astype(np.int32)
    s = scales[..., None]
    amax = np.abs(cg).max(-1)
    hits = np.where(amax > 0, np.abs(qg).max(-1) == 127, True)
    err_ok = np.abs(qg * s - cg) <= s / 2 * (1 + 1e-6)
    return np.abs(qg).max() <= 127 and hits.all() and err_ok.all()


@pytest.mark.parametrize("dt", ["f32", "f16", "bf16"])
def test_grouped_quantizer_oracle(golden, oracle, dt):
    """The per-32 absmax archive (no reference code; README.md:487-494):
    a one-group row equals the pinned row quantizer bit for bit; with
    groups of very different magnitude every group keeps its own absmax at
    +-127 and a half-step error bound (a planted mistake, one scale per row,
    breaks both); k = r round trips within the summed half steps."""
    rng = np.random.default_rng(11)
    r = 8
    basis = golden("basis").data["r8"]
    one = oracle.round_to(rng.standard_normal((2, 3, 40, 32)).astype(np.float32), dt)
    _, rc, rs = oracle.jpeg_encode(one, r, 4, basis[:4], dt, quant=True)
    _, gc, gs = oracle.jpeg_encode_grouped(one, r, 4, basis[:4], dt)
    assert gs.shape == rs.shape + (1,)
    assert np.array_equal(gc, rc) and np.array_equal(_bits(gs[..., 0]), _bits(rs))
    x = rng.standard_normal((2, 2, 43, 128)).astype(np.float32)
    x[..., 32:64] *= 100.0                        # one loud group per row
    x[..., 96:128] *= 1e-3                        # and one quiet one
    x = oracle.round_to(x, dt)
    coef, codes, scales = oracle.jpeg_encode_grouped(x, r, 4, basis[:4], dt)
    assert scales.shape == coef.shape[:-1] + (4,)
    assert _group_bounds_hold(coef, codes, scales, 32)
    _, row_codes, row_scales = oracle.jpeg_encode(x, r, 4, basis[:4], dt, quant=True)
    planted = np.repeat(row_scales[..., None], 4, axis=-1)
    assert not _group_bounds_hold(coef, row_codes, planted, 32)
    # quieter groups quantize finer: the grouped error is never above the row's
    deq_g = oracle.grouped_coefficients(codes, scales)
    deq_r = row_codes * row_scales[..., None]
    assert np.all(np.abs(deq_g - coef) <= np.abs(row_scales)[..., None] / 2 * (1 + 1e-6))
    assert np.abs(deq_g - coef)[..., 96:].max() < np.abs(deq_r - coef)[..., 96:].max()
    # k = r: the orthonormal synthesis of the dequantised rows is within
    # sum_j |basis[j, t]| * s_j / 2 of the (dtype-rounded) coefficients' view
    if dt == "f32":
        cf, cc, cs = oracle.jpeg_encode_grouped(x, r, r, basis, dt)
        rec = oracle.jpeg_decode(oracle.grouped_coefficients(cc, cs), r, basis, "f32")
        exact = oracle.jpeg_decode(cf, r, basis, "f32")
        half = np.repeat(cs, 32, axis=-1) / 2               # (..., n, r, D)
        bound = np.einsum("jt,...njd->...ntd", np.abs(basis), half)
        bound = bound.reshape(rec.shape) * (1 + 1e-5) + 1e-6
        assert np.all(np.abs(rec - exact) <= bound)
        assert np.abs(exact[..., :43, :] - x).max() < 1e-5 * np.abs(x).max()


# ---------------------------------------------------------------- png

def test_topk_keep_matches_torch_topk(oracle):
    rng = np.random.default_rng(5)
    for n in (3, 7, 15, 31, 63):
        for m in sorted({1, 2, max(1, n // 4), n // 2, n - 1}):
            for trial in range(60):
                kind = trial % 3
                if kind == 0:
                    v = rng.integers(0, 3, n).astype(np.float32)
                elif kind == 1:
                    v = (rng.integers(0, 6, n) * 0.5).astype(np.float32)
                else:
                    v = np.abs(rng.standard_normal(n)).astype(np.float32)
                col = torch.from_numpy(v).reshape(1, n, 1).repeat(1, 1, 2)
                idx = col.topk(m, dim=-2).indices[0, :, 0].numpy()
                ref = np.zeros(n, bool)
                ref[idx] = True
                assert np.array_equal(oracle.topk_keep(v, m), ref), (n, m, v)


def _png_cases():
    from tests.conftest import Golden
    return Golden("png").names()


@pytest.mark.parametrize("name", _png_cases())
def test_png_oracle_matches_reference(golden, oracle, name):
    G = golden("png")
    c, m = G.case(name), G.meta[name]
    dt, r, keep = m["dtype"], m["r"], m["keep"]
    x = oracle.values_of(c["x"], dt)
    d, a = oracle.png_encode(x, r, keep)
    assert np.array_equal(_bits(d), _bits(c["deltas"]))          # includes -0.0 signs
    assert np.array_equal(_bits(a), _bits(oracle.values_of(c["anchors"], dt)))
    rec = oracle.png_decode(d, a, dt)
    assert np.array_equal(_bits(rec), _bits(oracle.values_of(c["rec"], dt)))


@pytest.mark.parametrize("name", [n for n in _png_cases() if "_k1" not in n and "r32" not in n])
def test_png_pack_round_trip_on_reference_outputs(golden, oracle, name):
    """The packed Top-M archive holds png_filter's output exactly: unpacking
    the packing of the reference's own deltas (golden, -0.0 signs and tie
    columns included) gives them back bit for bit; every column keeps
    exactly keep_m slots."""
    G = golden("png")
    c, m = G.case(name), G.meta[name]
    keep_m = oracle.png_keep_m(m["r"], m["keep"])
    d = np.asarray(c["deltas"], np.float32)
    vals, mask = oracle.png_pack(d, keep_m)
    assert vals.shape == d.shape[:-2] + (keep_m, d.shape[-1])
    assert np.all(np.bitwise_count(mask & 0x7FFF) == keep_m)
    assert np.all((mask & (mask >> 16) & 0x7FFF) == 0)          # no sign bit on a kept step
    u = oracle.png_unpack(vals, mask, m["r"])
    assert np.array_equal(_bits(u), _bits(d))


def test_png_pack_exhaustive_small_columns(oracle):
    """Every column of 4 steps over {+0, -0, 1, -2, 3, NaN-free ties} with at
    most keep_m non-zero steps round-trips bit for bit, for keep_m 1..4;
    the kept set is the non-zero steps plus the lowest-index zeros."""
    import itertools
    alphabet = np.array([0.0, -0.0, 1.0, -2.0, 3.0, 1.0], np.float32)
    cols = np.array(list(itertools.product(range(len(alphabet)), repeat=4)))
    vals_all = alphabet[cols]                                     # (N, 4)
    nz = (vals_all.view(np.uint32) & 0x7FFFFFFF) != 0
    for keep_m in range(1, 5):
        ok = nz.sum(-1) <= keep_m
        d = vals_all[ok].T[None, :, :].copy()                     # (1 block, 4 steps, N)
        v, mask = oracle.png_pack(d, keep_m)
        assert np.array_equal(_bits(oracle.png_unpack(v, mask, 5)), _bits(d))
        kept = (mask[0][None, :] >> np.arange(4)[:, None]) & 1
        nzc = nz[ok].T
        assert np.all(kept[nzc] == 1)                             # non-zero steps kept
        fill = np.cumsum(kept * ~nzc, 0)                          # zeros kept, lowest first
        first_unkept = np.argmax((kept == 0) & ~nzc, axis=0)
        assert np.all((fill[-1] == keep_m - nzc.sum(0)))
        has = ((kept == 0) & ~nzc).any(0)
        for col in np.nonzero(has)[0][:50]:
            assert not np.any((kept[:, col] == 1) & ~nzc[:, col] & (np.arange(4) > first_unkept[col]))
    with pytest.raises(ValueError):
        oracle.png_pack(np.ones((1, 4, 2), np.float32), 2)       # 4 non-zero steps, keep_m 2


def test_png_pack_planted_mistakes_are_caught(oracle):
    """The round-trip check sees the mistakes a packer could make: sign
    words dropped (pruned -0.0 come back as +0.0) and slot values shifted by
    one rank."""
    x = oracle.ar1((1, 2, 16 * 12, 32), 0.95, 3)
    d, _ = oracle.png_encode(x, 16, 0.25)
    vals, mask = oracle.png_pack(d, 4)
    assert np.array_equal(_bits(oracle.png_unpack(vals, mask, 16)), _bits(d))
    no_sign = mask & np.uint32(0xFFFF)
    assert not np.array_equal(_bits(oracle.png_unpack(vals, no_sign, 16)), _bits(d))
    shifted = np.roll(vals, 1, axis=-2)
    assert not np.array_equal(_bits(oracle.png_unpack(shifted, mask, 16)), _bits(d))
    # reconstruction through the dense decoder is the dense archive's own
    a = oracle.png_encode(x, 16, 0.25)[1]
    rec = oracle.png_decode(oracle.png_unpack(vals, mask, 16), a, "f32")
    assert np.array_equal(_bits(rec), _bits(oracle.png_decode(d, a, "f32")))


@pytest.mark.parametrize("name", _png_cases())
def test_torch_path_png_matches_reference(golden, name):
    """oracle/torch_path.py's png operations (bench.py's C4 CPU baseline)
    reproduce the reference's bits on this torch CPU build (Top-M tie order
    included)."""
    from oracle import torch_path as T
    G = golden("png")
    c, m = G.case(name), G.meta[name]
    dt = m["dtype"]
    x = _torch_of(c["x"], dt)
    d, a = T.png_filter(x, m["r"], m["keep"])
    assert np.array_equal(_bits(d.numpy()), _bits(c["deltas"]))
    assert np.array_equal(_bits(_np_of(a, dt)), _bits(c["anchors"]))
    rec = T.png_reconstruct(d, a)
    assert np.array_equal(_bits(_np_of(rec, dt)), _bits(c["rec"]))


def test_png_closed_form_properties(oracle):
    rng = np.random.default_rng(11)
    x = rng.standard_normal((2, 2, 64, 32)).astype(np.float32)
    # keep=1: bf16 round trip is bitwise (bf16 deltas are exact in fp32);
    # fp32 is lossless up to the fp32 rounding of anchor + prefix sum
    xb = oracle.round_to(x, "bf16")
    d, a = oracle.png_encode(xb, 8, 1.0)
    assert np.array_equal(_bits(oracle.png_decode(d, a, "bf16")), _bits(xb))
    d, a = oracle.png_encode(x, 8, 1.0)
    assert np.abs(oracle.png_decode(d, a, "f32") - x).max() < 1e-6
    # Top-M on tie-free data keeps exactly the m largest |delta| per column
    d, a = oracle.png_encode(x, 16, 0.25)
    full, _ = oracle.png_encode(x, 16, 1.0)
    m = math.ceil(15 * 0.25)
    kept = d != 0
    assert np.all(kept.sum(-2) == m)
    order = np.argsort(-np.abs(full), axis=-2, kind="stable")[..., :m, :]
    want = np.zeros_like(kept)
    np.put_along_axis(want, order, True, axis=-2)
    assert np.array_equal(kept, want)
    assert np.array_equal(d[kept], full[kept])


# ---------------------------------------------------------------- stream

def _stream_cases():
    from tests.conftest import Golden
    return Golden("stream").names()


@pytest.mark.parametrize("name", _stream_cases())
def test_stream_archive_is_blockwise_encode(golden, oracle, name):
    """_CodecStream.append (token by token, in chunks or in bulk) archives
    exactly the blockwise encode of the complete blocks; read() is their
    decode followed by the raw tail; crop(-5) is an exact truncation."""
    G = golden("stream")
    c, m = G.case(name), G.meta[name]
    cfg, dt = m["cfg"], m["dtype"]
    r = cfg["block_size"]
    x = oracle.values_of(c["x"], dt)
    S = x.shape[-2]
    n = S // r
    head = x[..., :n * r, :]
    if cfg["mode"] == "jpeg":
        k = cfg["keep_freqs"]
        basis = golden("basis").data[f"r{r}"][:k]
        if cfg.get("quant_bits"):
            _, codes, scales = oracle.jpeg_encode(head, r, k, basis, dt, quant=True)
            assert np.array_equal(codes, c["coeffs"])
            assert np.array_equal(_bits(scales), _bits(c["scales"]))
            rec = oracle.jpeg_decode(None, r, basis, dt, codes=codes, scales=scales)
        else:
            coef = oracle.jpeg_encode(head, r, k, basis, dt)
            assert np.array_equal(_bits(coef), _bits(oracle.values_of(c["coeffs"], dt)))
            rec = oracle.jpeg_decode(coef, r, basis, dt)
    else:
        d, a = oracle.png_encode(head, r, cfg["keep_ratio"])
        assert np.array_equal(_bits(d), _bits(c["deltas"]))
        assert np.array_equal(_bits(a), _bits(oracle.values_of(c["anchors"], dt)))
        rec = oracle.png_decode(d, a, dt)
    read = oracle.values_of(c["read"], dt)
    assert np.array_equal(_bits(read[..., :n * r, :]), _bits(rec))
    assert np.array_equal(_bits(read[..., n * r:, :]), _bits(x[..., n * r:, :]))
    assert np.array_equal(_bits(oracle.values_of(c["read_crop5"], dt)), _bits(read[..., :-5, :]))


# ---------------------------------------------------------------- attention

def _attn_cases():
    from tests.conftest import Golden
    return Golden("attention").names()


def oracle_attention_inputs(oracle, golden, c, m):
    """Oracle archive rows + raw tails of a golden attention case."""
    cfg, dt = m["cfg"], m["dtype"]
    r = cfg["block_size"]
    k = oracle.values_of(c["k"], dt)
    v = oracle.values_of(c["v"], dt)
    S = k.shape[-2]
    n = S // r
    rows = []
    for x in (k, v):
        head = x[..., :n * r, :]
        if cfg["mode"] == "jpeg":
            kk = cfg["keep_freqs"]
            basis = golden("basis").data[f"r{r}"][:kk]
            if cfg.get("quant_bits"):
                _, codes, scales = oracle.jpeg_encode(head, r, kk, basis, dt, quant=True)
                rows.append(oracle.stored_rows_jpeg(codes, scales))
            else:
                rows.append(oracle.stored_rows_jpeg(oracle.jpeg_encode(head, r, kk, basis, dt)))
            A = oracle.synthesis_matrix("jpeg", r, basis)
        else:
            d, a = oracle.png_encode(head, r, cfg["keep_ratio"])
            rows.append(oracle.stored_rows_png(d, a))
            A = oracle.synthesis_matrix("png", r)
    q = oracle.values_of(c["q"], dt)[:, :, 0]
    raw_k = k[..., n * r:, :] if S > n * r else None
    raw_v = v[..., n * r:, :] if S > n * r else None
    return q, rows[0], rows[1], raw_k, raw_v, A


@pytest.mark.parametrize("name", _attn_cases())
def test_attention_oracle_matches_reference_torch_path(golden, oracle, name):
    G = golden("attention")
    c, m = G.case(name), G.meta[name]
    q, rk, rv, zk, zv, A = oracle_attention_inputs(oracle, golden, c, m)
    D = m["D"]
    ref = oracle.values_of(c["out"], m["dtype"])[:, :, 0]
    got = oracle.attention(q, rk, rv, zk, zv, A, D ** -0.5)
    if m["dtype"] == "f32":
        assert np.abs(got - ref).max() < 1e-5
    else:
        # the reference's torch path runs its einsums in the query dtype
        assert np.abs(got - ref).max() <= 2e-3 * max(np.abs(ref).max(), 1e-3)


def test_attention_oracle_matches_dense_softmax_on_reconstruction(golden, oracle):
    """The coefficient-domain definition equals softmax(q K^T) V on the
    reconstructed tokens (jpeg int8, G=2, 3-token tail)."""
    G = golden("attention")
    name = "jpeg_i8_f32_g2_t3"
    c, m = G.case(name), G.meta[name]
    q, rk, rv, zk, zv, A = oracle_attention_inputs(oracle, golden, c, m)
    D, g = m["D"], m["G"]
    toks_k = np.concatenate([np.einsum("ps,bhnsd->bhnpd", A, rk).reshape(
        rk.shape[0], rk.shape[1], -1, D), zk], axis=2)
    toks_v = np.concatenate([np.einsum("ps,bhnsd->bhnpd", A, rv).reshape(
        rv.shape[0], rv.shape[1], -1, D), zv], axis=2)
    kk = np.repeat(toks_k, g, axis=1)
    vv = np.repeat(toks_v, g, axis=1)
    logits = np.einsum("bhd,bhtd->bht", q.astype(np.float64), kk) / math.sqrt(D)
    p = np.exp(logits - logits.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    dense = np.einsum("bht,bhtd->bhd", p, vv)
    got = oracle.attention(q, rk, rv, zk, zv, A, D ** -0.5)
    assert np.abs(got - dense).max() < 1e-10


def _torch_path_inputs(oracle, golden, c, m):
    """torch CPU tensors of a golden attention case as the reference's torch
    path sees them: stored rows in the work dtype, raw tails, A (r x s)."""
    import torch
    from tests.conftest import to_torch
    from oracle import torch_path
    cfg, dt = m["cfg"], m["dtype"]
    r = cfg["block_size"]
    q = to_torch(c["q"], dt, device="cpu")
    seqs = [oracle.values_of(c[x], dt) for x in ("k", "v")]
    S = seqs[0].shape[-2]
    n = S // r
    rows = []
    for x in seqs:
        head = x[..., :n * r, :]
        if cfg["mode"] == "jpeg":
            kk = cfg["keep_freqs"]
            basis = golden("basis").data[f"r{r}"][:kk]
            if cfg.get("quant_bits"):
                _, codes, scales = oracle.jpeg_encode(head, r, kk, basis, dt, quant=True)
                rows.append(torch_path.jpeg_rows(torch.from_numpy(codes),
                                                 torch.from_numpy(scales)[..., None], q.dtype))
            else:
                coef = oracle.jpeg_encode(head, r, kk, basis, dt)
                rows.append(to_torch(oracle.encode_as(coef, dt), dt, device="cpu"))
            A = torch.from_numpy(np.ascontiguousarray(basis)).t()
        else:
            d, a = oracle.png_encode(head, r, cfg["keep_ratio"])
            rows.append(torch_path.png_rows(torch.from_numpy(d),
                                            to_torch(oracle.encode_as(a, dt), dt, device="cpu")))
            A = torch.tril(torch.ones(r, r))
    raws = [None if S == n * r else to_torch(c[x], dt, device="cpu")[..., n * r:, :]
            for x in ("k", "v")]
    return q, rows[0], rows[1], raws[0], raws[1], A


@pytest.mark.parametrize("name", _attn_cases())
def test_torch_path_restatement_matches_reference(golden, oracle, name):
    """oracle/torch_path.py (bench.py's CPU baseline) reproduces the
    reference's impl="torch" outputs bit for bit on the golden cases, and
    agrees with the fp64 oracle within tolerance."""
    from oracle import torch_path
    G = golden("attention")
    c, m = G.case(name), G.meta[name]
    q, rk, rv, zk, zv, A = _torch_path_inputs(oracle, golden, c, m)
    out = torch_path.decode_attention(q, rk, rv, zk, zv, A, m["D"] ** -0.5)
    ref = c["out"]
    got = out.numpy() if m["dtype"] != "bf16" else out.view(torch.int16).numpy().view(np.uint16)
    assert got.dtype == ref.dtype and np.array_equal(got, ref)
    q64, rk64, rv64, zk64, zv64, A64 = oracle_attention_inputs(oracle, golden, c, m)
    exact = oracle.attention(q64, rk64, rv64, zk64, zv64, A64, m["D"] ** -0.5)
    vals = oracle.values_of(got, m["dtype"])[:, :, 0]
    tol = 1e-5 if m["dtype"] == "f32" else 4e-3 * np.abs(exact).max()
    assert np.abs(vals - exact).max() <= tol


def test_torch_path_restatement_catches_a_dropped_tail(golden, oracle):
    """A planted mistake (the raw tail left out) moves the restatement's
    output off the reference's bits."""
    from oracle import torch_path
    G = golden("attention")
    name = "jpeg_i8_f16_g4_t5"
    c, m = G.case(name), G.meta[name]
    q, rk, rv, zk, zv, A = _torch_path_inputs(oracle, golden, c, m)
    out = torch_path.decode_attention(q, rk, rv, None, None, A, m["D"] ** -0.5)
    assert not np.array_equal(out.numpy(), c["out"])
