"""GPU: archive / reconstruction kernels bit-exact against the reference's
golden vectors and against the oracle on seeded inputs (dtypes, block sizes,
feature widths, strides, padding, zero blocks, Top-M ties)."""

import math

import numpy as np
import pytest
import torch

import flashcodec_amd as fc
from tests.conftest import Golden, bits, seed_of, to_torch, to_values, torch_dtype

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.mark.parametrize("name", Golden("jpeg").names())
def test_jpeg_kernels_match_reference_bits(name, oracle):
    G = Golden("jpeg")
    c, m = G.case(name), G.meta[name]
    dt, r, k, S = m["dtype"], m["r"], m["k"], m["shape"][-2]
    print(f"case jpeg/{name}", flush=True)
    x = to_torch(c["x"], dt)
    coef = fc.dct_compress(x, r, k)
    assert coef.dtype == x.dtype
    assert np.array_equal(bits(to_values(coef)), bits(oracle.values_of(c["coef"], dt)))
    q, s = fc.quantize_coeffs(coef)
    assert q.dtype == torch.int8 and s.shape == coef.shape[:-1] + (1,)
    assert np.array_equal(q.cpu().numpy(), c["codes"])
    assert np.array_equal(bits(s[..., 0].cpu().numpy()), bits(c["scales"]))
    deq = fc.dequantize_coeffs(q, s)
    assert np.array_equal(bits(deq.cpu().numpy()), bits(c["deq_f32"]))
    deq_t = fc.dequantize_coeffs(q, s, torch_dtype(dt))
    assert np.array_equal(bits(to_values(deq_t)), bits(oracle.values_of(c["deq_T"], dt)))
    rec = fc.dct_decompress(coef, r, out_len=S)
    assert rec.dtype == torch.float32 and rec.shape == x.shape
    assert np.array_equal(bits(rec.cpu().numpy()), bits(c["rec"]))
    codec = fc.JPEGCodec(block_size=r, keep_freqs=k, quant_bits=8)
    rec_q = codec.decompress(q, out_len=S, scales=s)
    assert np.array_equal(bits(rec_q.cpu().numpy()), bits(c["rec_q"]))


@pytest.mark.parametrize("name", Golden("png").names())
def test_png_kernels_match_reference_bits(name, oracle):
    G = Golden("png")
    c, m = G.case(name), G.meta[name]
    dt, r, keep = m["dtype"], m["r"], m["keep"]
    print(f"case png/{name}", flush=True)
    x = to_torch(c["x"], dt)
    d, a = fc.png_filter(x, r, keep)
    assert d.dtype == torch.float32 and a.dtype == x.dtype
    assert np.array_equal(bits(d.cpu().numpy()), bits(c["deltas"]))
    assert np.array_equal(bits(to_values(a)), bits(oracle.values_of(c["anchors"], dt)))
    rec = fc.png_reconstruct(d, a)
    assert np.array_equal(bits(to_values(rec)), bits(oracle.values_of(c["rec"], dt)))


JPEG_RANDOM = [
    # dtype, r, k, (B, H, S, D)
    ("f16", 8, 4, (4, 8, 256, 128)),
    ("bf16", 8, 2, (2, 8, 203, 128)),
    ("f32", 8, 8, (2, 4, 64, 256)),
    ("f16", 16, 4, (1, 4, 160, 64)),
    ("f32", 4, 3, (2, 2, 40, 36)),      # D % 8 != 0: 4-wide lanes
    ("bf16", 8, 4, (1, 2, 64, 7)),      # odd D: scalar lanes
    ("f16", 24, 5, (1, 2, 96, 48)),     # streaming path (r > 16)
    ("f32", 64, 8, (1, 1, 130, 32)),    # largest block
    ("bf16", 2, 1, (3, 1, 9, 512)),     # widest head
]


def _oracle_jpeg(oracle, x_vals, r, k, dt):
    basis = fc.dct_basis(r, k).numpy()
    return oracle.jpeg_encode(x_vals, r, k, basis, dt, quant=True), basis


@pytest.mark.parametrize("dt,r,k,shape", JPEG_RANDOM)
def test_jpeg_kernels_match_oracle(dt, r, k, shape, oracle):
    print(f"case jpeg-random {dt} r={r} k={k} shape={shape}", flush=True)
    rng = np.random.default_rng(seed_of(dt, r, k, shape))
    xv = oracle.round_to(oracle.ar1(shape, 0.9, 1) * np.exp(rng.uniform(-3, 3, shape[:-2] + (1, shape[-1]))).astype(np.float32), dt)
    x = torch.from_numpy(xv).to(torch_dtype(dt)).to(DEV)
    (coef, codes, scales), basis = _oracle_jpeg(oracle, xv, r, k, dt)
    got = fc.dct_compress(x, r, k)
    assert np.array_equal(bits(to_values(got)), bits(coef))
    q, s = fc.quantize_coeffs(got)
    assert np.array_equal(q.cpu().numpy(), codes)
    assert np.array_equal(bits(s[..., 0].cpu().numpy()), bits(scales))
    S = shape[-2]
    rec = fc.dct_decompress(got, r, out_len=S)
    assert np.array_equal(bits(rec.cpu().numpy()), bits(oracle.jpeg_decode(coef, r, basis)[..., :S, :]))
    # strided input: rows of a wider buffer (token stride D + 8)
    wide = torch.zeros(shape[:-1] + (shape[-1] + 8,), dtype=x.dtype, device=DEV)
    wide[..., :shape[-1]] = x
    xt = wide[..., :shape[-1]]
    assert not xt.is_contiguous() and xt.stride(-1) == 1
    assert torch.equal(fc.dct_compress(xt, r, k), got)


PNG_RANDOM = [
    ("f32", 16, 0.25, (2, 8, 512, 128), "ar1"),
    ("f32", 16, 1.0, (2, 4, 256, 128), "ar1"),
    ("bf16", 8, 0.5, (2, 4, 200, 64), "ties"),
    ("f16", 16, 0.25, (1, 4, 256, 32), "ties"),
    ("f32", 12, 0.3, (1, 2, 100, 40), "ties"),
    ("f32", 32, 0.2, (1, 2, 128, 16), "ties"),
    ("bf16", 64, 0.1, (1, 1, 192, 8), "ties"),
    ("f32", 2, 0.5, (2, 2, 33, 24), "ar1"),
    ("f16", 8, 0.25, (1, 2, 64, 5), "ties"),
]


@pytest.mark.parametrize("dt,r,keep,shape,kind", PNG_RANDOM)
def test_png_kernels_match_oracle(dt, r, keep, shape, kind, oracle):
    print(f"case png-random {dt} r={r} keep={keep} shape={shape} {kind}", flush=True)
    rng = np.random.default_rng(seed_of(dt, r, keep, shape))
    if kind == "ties":
        xv = (rng.integers(-6, 7, shape) / 8.0).astype(np.float32)
    else:
        xv = oracle.ar1(shape, 0.98, 3)
    xv = oracle.round_to(xv, dt)
    x = torch.from_numpy(xv).to(torch_dtype(dt)).to(DEV)
    d_ref, a_ref = oracle.png_encode(xv, r, keep)
    d, a = fc.png_filter(x, r, keep)
    assert np.array_equal(bits(d.cpu().numpy()), bits(d_ref))
    assert np.array_equal(bits(to_values(a)), bits(a_ref))
    rec = fc.png_reconstruct(d, a)
    assert np.array_equal(bits(to_values(rec)), bits(oracle.png_decode(d_ref, a_ref, dt)))


def test_png_bf16_lossless_and_pruning_counts():
    torch.manual_seed(0)
    x = torch.randn(2, 4, 64, 32, device=DEV).to(torch.bfloat16)
    d, a = fc.png_filter(x, 8, 1.0)
    assert torch.equal(fc.png_reconstruct(d, a)[..., :64, :], x)
    xs = torch.cumsum(torch.randn(2, 4, 64, 32, device=DEV) * 0.1, dim=-2)
    d, a = fc.png_filter(xs, 16, 0.25)
    assert int((d != 0).sum(-2).max()) <= math.ceil(15 * 0.25)
    err1 = (fc.png_reconstruct(*fc.png_filter(xs, 8, 1.0)) - xs).abs().mean()
    err05 = (fc.png_reconstruct(*fc.png_filter(xs, 8, 0.5)) - xs).abs().mean()
    assert err05 > err1


def test_dct_autograd_and_shapes():
    x = torch.randn(2, 3, 50, 16, device=DEV, requires_grad=True)
    rec = fc.dct_decompress(fc.dct_compress(x, 8, 2), 8, out_len=50)
    assert rec.shape == x.shape
    rec.pow(2).mean().backward()
    assert x.grad is not None and torch.isfinite(x.grad).all()
    # gradient of the orthogonal projection P = M^T M (per block): dL/dx = P dL/drec
    g = 2 * rec.detach() / rec.numel()
    xp = torch.nn.functional.pad(g, (0, 0, 0, 6)).reshape(2, 3, 7, 8, 16)
    M = fc.dct_basis(8, 2).to(DEV).double()
    P = M.t() @ M
    want = torch.einsum("ts,bhnsd->bhntd", P, xp.double()).reshape(2, 3, 56, 16)[..., :50, :]
    assert torch.allclose(x.grad.double(), want, atol=1e-6)
    flat = torch.randn(100, 16, device=DEV)
    assert fc.dct_decompress(fc.dct_compress(flat, 8, 2), 8, 100).shape == flat.shape


def test_jpeg_quality_properties():
    torch.manual_seed(0)
    B, H, S, D, R = 2, 4, 64, 32, 8
    x = torch.randn(B, H, S, D, device=DEV)
    assert (fc.dct_decompress(fc.dct_compress(x, R, R), R, S) - x).abs().max() < 1e-5
    smooth = torch.cumsum(torch.randn(B, H, S, D, device=DEV) * 0.1, dim=-2)
    rec = fc.dct_decompress(fc.dct_compress(smooth, R, 2), R, S)
    cos = torch.nn.functional.cosine_similarity(rec.flatten(), smooth.flatten(), dim=0)
    assert cos > 0.99
    e2 = (fc.dct_decompress(fc.dct_compress(smooth, R, 2), R, S) - smooth).abs().mean()
    e4 = (fc.dct_decompress(fc.dct_compress(smooth, R, 4), R, S) - smooth).abs().mean()
    assert e4 < e2


def _dtype_values(dt):
    """Every finite value of f16 / bf16, as float32."""
    b = np.arange(1 << 16, dtype=np.uint32)
    vals = (b << 16).view(np.float32) if dt == "bf16" else \
        b.astype(np.uint16).view(np.float16).astype(np.float32)
    return vals[np.isfinite(vals)]


def _near_tie_rows(dt, rng, D=64):
    """Quantizer rows whose quotients c / s sit on or a few ulp beside the
    half-integers where rint changes value: element 0 of each row is the row
    maximum amax (so s = T(amax / 127)), the others are ((n + 1/2) s) nudged
    by -3..3 ulp for f32; for f16 / bf16 every finite value of the dtype with
    |c| <= amax.  Scales span normal, tiny and subnormal magnitudes (1 / s
    overflows for the last)."""
    rows = []
    if dt == "f32":
        amaxes = [np.float32(v) for v in np.exp2(rng.uniform(-40, 40, 96))]
        amaxes += [np.float32(127 * 2.0 ** e * (1 + j / 16)) for e in (-20, -3, 0, 5) for j in range(16)]
        amaxes += [np.float32(1e-37), np.float32(3e-39), np.float32(1e-44)]
        for amax in amaxes:
            s = np.float32(amax) / np.float32(127)
            n = rng.integers(-127, 127, D - 1).astype(np.float64)
            c = ((n + 0.5) * np.float64(s)).astype(np.float32)
            ib = c.view(np.int32) + rng.integers(-3, 4, D - 1).astype(np.int32)
            c = np.where(c == 0, c, ib.view(np.float32))
            c = np.clip(c, -amax, amax)
            rows.append(np.concatenate([[amax], c]).astype(np.float32))
    else:
        vals = _dtype_values(dt)
        for amax in (1.5, 0.009765625, 300.0, 127 / 16, 127 * 8):
            amax = np.float32(amax)
            sel = vals[np.abs(vals) <= amax]
            pad = (-len(sel)) % (D - 1)
            sel = np.concatenate([sel, np.zeros(pad, np.float32)]).reshape(-1, D - 1)
            rows.append(np.concatenate([np.full((len(sel), 1), amax, np.float32), sel], 1))
    return np.vstack([np.atleast_2d(r) for r in rows]).astype(np.float32)


@pytest.mark.parametrize("dt", ["f32", "f16", "bf16"])
def test_quantizer_near_half_integer_quotients(dt, oracle):
    """Codes and scales of quantize_coeffs and of the fused int8 archive
    kernel stay bit-identical to the IEEE-quotient quantizer on the inputs
    where a reciprocal-multiply shortcut would round the other way."""
    from flashcodec_amd.codecs import jpeg as jp
    print(f"case quant-ties {dt}", flush=True)
    rng = np.random.default_rng(seed_of("quant-ties", dt))
    rows = _near_tie_rows(dt, rng)
    R, D = rows.shape
    codes, scales = oracle.quantize(rows, dt)
    # the rows do sit where a bare rint(c * fl(1 / s)) picks other codes (f32)
    # or hit exact ties (all dtypes)
    with np.errstate(over="ignore", invalid="ignore", divide="ignore"):
        x = rows * (np.float32(1) / scales.astype(np.float32))[:, None]
        bare = np.clip(np.rint(x), -127, 127)
        assert (np.abs(np.abs(x - np.rint(x)) - 0.5) < 2.0 ** -15).sum() > 100
    if dt == "f32":
        assert (bare != codes).sum() > 100
    assert np.array_equal(oracle.round_to(rows, dt), rows)  # representable in dt
    t = torch.from_numpy(rows).to(torch_dtype(dt)).to(DEV)
    q, s = fc.quantize_coeffs(t)
    assert np.array_equal(q.cpu().numpy(), codes)
    assert np.array_equal(bits(s[..., 0].cpu().numpy()), bits(scales))
    # fused archive kernel, r = k = 1: the coefficient is the token itself
    x4 = t.reshape(1, 1, R, D)
    cq = torch.zeros((1, 1, R, 1, D), dtype=torch.int8, device=DEV)
    cs = torch.zeros((1, 1, R, 1, 1), dtype=torch.float32, device=DEV)
    jp.encode_into(x4, 1, 1, 8, cq, cs, R, 0, R, R)
    assert np.array_equal(cq.reshape(R, D).cpu().numpy(), codes)
    assert np.array_equal(bits(cs.reshape(R).cpu().numpy()), bits(scales))


def _near_tie_blocks(dt, rng, D=64):
    """8-token blocks whose only nonzero token is the first, so the freq-0
    DCT coefficient is fl(v w0) (w0 = basis[0][0]); v is picked per element
    so that these coefficients sit on or a few ulp beside half-integer
    multiples of the row's scale (f32), or runs over every finite dtype
    value in a range (f16 / bf16)."""
    w0 = np.float32(fc.dct_basis(8, 4).numpy()[0, 0])
    rows = []
    if dt == "f32":
        for vmax in np.exp2(rng.uniform(-30, 30, 160)).astype(np.float32):
            amax = np.float32(vmax * w0)
            s = amax / np.float32(127)
            n = rng.integers(-127, 127, D - 1).astype(np.float64)
            v = ((n + 0.5) * np.float64(s) / np.float64(w0)).astype(np.float32)
            vb = v.view(np.int32) + rng.integers(-3, 4, D - 1).astype(np.int32)
            v = np.clip(np.where(v == 0, v, vb.view(np.float32)), -vmax, vmax)
            rows.append(np.concatenate([[vmax], v]).astype(np.float32))
        rows = np.vstack(rows)
    else:
        # row maxima whose scale has at most 3 significant bits, so every
        # coefficient that is an odd multiple of a small power of two is an
        # exact tie
        from oracle import oracle as O
        allv = _dtype_values(dt)
        for e in (-4, 3, -10):
            target = np.float32(127 * 2.0 ** e / w0)
            cand = allv[(allv >= target / 2) & (allv <= target * 2)]
            sc = O.round_to(O.round_to(cand * w0, dt) / np.float32(127), dt)
            frac, _ = np.frexp(sc)
            vmax = cand[(frac * 8) == np.round(frac * 8)][0]
            sel = allv[np.abs(allv) <= vmax]
            pad = (-len(sel)) % (D - 1)
            sel = np.concatenate([sel, np.zeros(pad, np.float32)]).reshape(-1, D - 1)
            rows.append(np.concatenate([np.full((len(sel), 1), vmax, np.float32), sel], 1))
        rows = np.vstack(rows)
    R = rows.shape[0]
    x = np.zeros((1, 1, R * 8, D), np.float32)
    x[0, 0, ::8] = rows
    return x


@pytest.mark.parametrize("dt", ["f32", "f16", "bf16"])
def test_archive_r8_near_half_integer_quotients(dt, oracle):
    """The r = 8 int8 archive kernel (reciprocal codes, DPP row max, fma
    division for the scale) stays bit-identical to the IEEE-quotient
    quantizer on coefficients at and around rounding ties."""
    from flashcodec_amd.codecs import jpeg as jp
    print(f"case archive-r8-ties {dt}", flush=True)
    rng = np.random.default_rng(seed_of("archive-r8-ties", dt))
    xv = _near_tie_blocks(dt, rng)
    assert np.array_equal(oracle.round_to(xv, dt), xv)
    _, S, D = xv.shape[1:]
    m = S // 8
    basis = fc.dct_basis(8, 4).numpy()
    _, codes, scales = oracle.jpeg_encode(xv, 8, 4, basis, dt, quant=True)
    coef = oracle.jpeg_encode(xv, 8, 4, basis, dt)
    c0, s0 = coef[0, 0, :, 0], scales[0, 0, :, 0]
    with np.errstate(over="ignore", invalid="ignore", divide="ignore"):
        xq = c0 * (np.float32(1) / s0)[:, None]
        assert (np.abs(np.abs(xq - np.rint(xq)) - 0.5) < 2.0 ** -15).sum() > 100
        if dt == "f32":
            assert (np.clip(np.rint(xq), -127, 127) != codes[0, 0, :, 0]).sum() > 100
    x = torch.from_numpy(xv).to(torch_dtype(dt)).to(DEV)
    cq = torch.zeros((1, 1, m, 4, D), dtype=torch.int8, device=DEV)
    cs = torch.zeros((1, 1, m, 4, 1), dtype=torch.float32, device=DEV)
    jp.encode_into(x, 8, 4, 8, cq, cs, m, 0, m, S)
    assert np.array_equal(cq.cpu().numpy(), codes)
    assert np.array_equal(bits(cs[..., 0].cpu().numpy()), bits(scales))


def _double_rounding_blocks(rng, n_blocks=1 << 20):
    """f16 8-token blocks whose DCT coefficient (r = 8, k = 4), an fma chain
    in fp32, lands exactly on an f16 halfway point while the exact value of
    the last fma does not: fp32-then-f16 rounding (the reference's) and a
    single rounding to f16 then give neighbouring f16 values.  Returns
    (blocks (n, 8) f32 values, freq, correct f16 value, single-rounded)."""
    w = fc.dct_basis(8, 4).numpy().astype(np.float64)
    x = (rng.standard_normal((n_blocks, 8)) * rng.uniform(0.1, 10, (n_blocks, 1)))
    x = x.astype(np.float16).astype(np.float64)
    out = []
    for j in range(4):
        acc = np.zeros(n_blocks)
        exact = np.ones(n_blocks, bool)
        for t in range(8):
            p = x[:, t] * w[j, t]                  # exact: 11 x 24 bits
            e = p + acc
            exact &= ((e - acc) == p) & ((e - p) == acc)
            if t < 7:
                acc = e.astype(np.float32).astype(np.float64)
        good = e.astype(np.float32).astype(np.float16).astype(np.float64)
        single = e.astype(np.float16).astype(np.float64)
        for i in np.nonzero(exact & (good != single))[0]:
            out.append((x[i].astype(np.float32), j, good[i], single[i]))
    return out


def test_f16_coefficients_round_through_fp32(oracle):
    """f16 coefficients are the fp32 fma chain rounded to f16 (two
    roundings), never a fused single rounding: checked on blocks where the
    two differ, for dct_compress and for the r = 8 int8 archive kernel
    (rows built so the correct coefficient sits exactly on a code tie)."""
    from flashcodec_amd.codecs import jpeg as jp
    print("case f16-double-rounding", flush=True)
    rng = np.random.default_rng(seed_of("f16-double-rounding"))
    hits = _double_rounding_blocks(rng)
    assert len(hits) > 100
    w = fc.dct_basis(8, 4).numpy()
    f16 = _dtype_values("f16")
    f16 = f16[f16 > 0]
    blocks, expect_flip = [], 0
    for xb, j, good, single in hits:
        # scale s with good / s = n + 1/2 exactly (an odd divisor d of the
        # significand M of |good|, n = (d - 1) / 2 <= 126)
        mant, ex = np.frexp(abs(good))
        M, e2 = int(mant * 2048), int(ex) - 11
        while M % 2 == 0:
            M, e2 = M // 2, e2 + 1
        d = max([dd for dd in range(1, 254, 2) if M % dd == 0])
        s = np.float32(2.0 * abs(good) / d)
        if s < 2.0 ** -14 or oracle.round_to(np.array([s]), "f16")[0] != s:
            continue
        # a block whose only token gives freq-j coefficient A with
        # f16(A / 127) == s: the row's absmax, so the row scale is s
        tgt = 127 * float(s) / abs(float(w[j, 0]))
        cand = f16[(f16 > tgt * 0.98) & (f16 < tgt * 1.02)]
        coefs = oracle.round_to((cand * np.float32(abs(w[j, 0]))).astype(np.float32), "f16")
        sc = oracle.round_to(coefs / np.float32(127), "f16")
        ok = (sc == s) & (coefs >= abs(good))
        if not ok.any():
            continue
        v = cand[ok][0] * np.sign(w[j, 0])
        blk = np.zeros((8, 8), np.float32)
        blk[:, 0] = xb
        blk[0, 1] = v
        blocks.append(blk)
        q_good = np.rint(np.float32(good) / s)
        q_single = np.rint(np.float32(single) / s)
        expect_flip += int(q_good != q_single)
        if len(blocks) == 64:
            break
    assert len(blocks) >= 32 and expect_flip >= 8
    xv = np.concatenate(blocks)[None, None]           # (1, 1, 8n, 8)
    x = torch.from_numpy(xv).to(torch.float16).to(DEV)
    basis = fc.dct_basis(8, 4).numpy()
    coef, codes, scales = oracle.jpeg_encode(xv, 8, 4, basis, "f16", quant=True)
    got = fc.dct_compress(x, 8, 4)
    assert np.array_equal(bits(to_values(got)), bits(coef))
    m = len(blocks)
    cq = torch.zeros((1, 1, m, 4, 8), dtype=torch.int8, device=DEV)
    cs = torch.zeros((1, 1, m, 4, 1), dtype=torch.float32, device=DEV)
    jp.encode_into(x, 8, 4, 8, cq, cs, m, 0, m, 8 * m)
    assert np.array_equal(bits(cs[..., 0].cpu().numpy()), bits(scales))
    assert np.array_equal(cq.cpu().numpy(), codes)


@pytest.mark.parametrize("dt", ["f32", "f16", "bf16"])
def test_quantizer_nan_and_inf(dt, oracle):
    """NaN coefficients get code 0 and leave the row's absmax alone; an
    infinite coefficient makes the scale infinite (codes 0), in the row
    quantizer and in both int8 archive kernels (r = 1 general, r = 8)."""
    from flashcodec_amd.codecs import jpeg as jp
    print(f"case quant-nan-inf {dt}", flush=True)
    rng = np.random.default_rng(seed_of("quant-nan-inf", dt))
    D, R = 64, 48
    rows = oracle.round_to(rng.standard_normal((R, D)).astype(np.float32) * 3, dt)
    for i in range(0, R, 3):
        rows[i, rng.integers(0, D, 3)] = np.nan
    rows[5, 7] = np.inf
    rows[11, 0] = -np.inf
    codes, scales = oracle.quantize(rows, dt)
    assert (codes[np.isnan(rows)] == 0).all()
    t = torch.from_numpy(rows).to(torch_dtype(dt)).to(DEV)
    q, s = fc.quantize_coeffs(t)
    assert np.array_equal(q.cpu().numpy(), codes)
    assert np.array_equal(bits(s[..., 0].cpu().numpy()), bits(scales))
    # r = 1 (general kernel) and r = 8 (token 0 of each block carries the row)
    for r in (1, 8):
        xv = np.zeros((1, 1, R * r, D), np.float32)
        xv[0, 0, ::r] = rows
        k = 1 if r == 1 else 4
        basis = fc.dct_basis(r, k).numpy()
        _, codes_r, scales_r = oracle.jpeg_encode(xv, r, k, basis, dt, quant=True)
        x = torch.from_numpy(xv).to(torch_dtype(dt)).to(DEV)
        cq = torch.zeros((1, 1, R, k, D), dtype=torch.int8, device=DEV)
        cs = torch.zeros((1, 1, R, k, 1), dtype=torch.float32, device=DEV)
        jp.encode_into(x, r, k, 8, cq, cs, R, 0, R, R * r)
        assert np.array_equal(cq.cpu().numpy(), codes_r), r
        assert np.array_equal(bits(cs[..., 0].cpu().numpy()), bits(scales_r)), r
