"""GPU: materialisation-free decode attention against the fp64 oracle, the
reference's torch-path outputs (golden) and dense attention on the
reconstructed view.

Tolerances (the contract's): fp32 outputs within 1e-5 absolute; fp16 / bf16
outputs within 2e-3 * max|ref| plus half an ulp of the output dtype at each
element (the final rounding the output dtype forces).
"""

import math

import numpy as np
import pytest
import torch

import flashcodec_amd as fc
from flashcodec_amd.cache import _CodecStream
from tests.conftest import Golden, seed_of, to_torch, to_values, torch_dtype

pytestmark = pytest.mark.gpu
DEV = "cuda"
HALF_ULP = {"f16": 2.0 ** -11, "bf16": 2.0 ** -8}


def assert_close(out, ref, dt):
    out = np.asarray(out, np.float64)
    ref = np.asarray(ref, np.float64)
    err = np.abs(out - ref)
    if dt == "f32":
        assert err.max() <= 1e-5, f"max abs err {err.max():.3e}"
    else:
        tol = 2e-3 * np.abs(ref).max() + HALF_ULP[dt] * np.abs(ref)
        bad = err > tol
        assert not bad.any(), f"{bad.sum()} elements out of tolerance; max err {err.max():.3e}"


def assert_close_pair(a, b, dt):
    """Two outputs of the same attention that were each rounded to the
    output dtype once: the contract's 2e-3 of max|b| plus a whole ulp (half
    an ulp per rounding) at each element."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    err = np.abs(a - b)
    if dt == "f32":
        assert err.max() <= 2e-5, f"max abs err {err.max():.3e}"
    else:
        tol = 2e-3 * np.abs(b).max() + 2 * HALF_ULP[dt] * np.abs(b)
        bad = err > tol
        assert not bad.any(), f"{bad.sum()} elements out of tolerance; max err {err.max():.3e}"


def stream_rows(oracle, st):
    """fp64 stored rows of a stream, read from its device buffers."""
    n = st.n_blocks
    if st.codec.name == "jpeg":
        c = st._coeffs[:, :, :n].float().cpu().numpy()
        if st.codec.quantized:
            sc = st._scales[:, :, :n].cpu().numpy()
            return oracle.stored_rows_jpeg(c, sc if st.codec.quant_group else sc[..., 0])
        return oracle.stored_rows_jpeg(c)
    if st.codec.packed:
        d = oracle.png_unpack(st._packed[:, :, :n].cpu().numpy(),
                              st._packed_mask[:, :, :n].cpu().numpy().view(np.uint32),
                              st.block_size)
    else:
        d = st._deltas[:, :, :n].cpu().numpy()
    return oracle.stored_rows_png(d, st._anchors[:, :, :n].float().cpu().numpy())


def oracle_out(oracle, q, ks, vs, scale):
    c = ks.codec
    r = ks.block_size
    if c.name == "jpeg":
        A = oracle.synthesis_matrix("jpeg", r, fc.dct_basis(r, c.keep_freqs).numpy())
    else:
        A = oracle.synthesis_matrix("png", r)
    if ks.n_blocks:
        rk, rv = stream_rows(oracle, ks), stream_rows(oracle, vs)
    else:
        Bq, Hk, D = q.shape[0], (ks.raw.shape[1]), q.shape[-1]
        s = c.keep_freqs if c.name == "jpeg" else r
        rk = rv = np.zeros((Bq, Hk, 0, s, D))
    zk = None if ks.raw is None else to_values(ks.raw)
    zv = None if vs.raw is None else to_values(vs.raw)
    return oracle.attention(to_values(q)[:, :, 0], rk, rv, zk, zv, A, scale, n_threads=8)


def build_streams(cfg, dt, B, Hk, S, D, seed, oracle, feed="bulk"):
    rng = np.random.default_rng(seed)
    sc = np.exp(rng.uniform(-1, 1, (B, Hk, 1, D))).astype(np.float32)
    k = torch.from_numpy(oracle.ar1((B, Hk, S, D), 0.95, seed) * sc).to(torch_dtype(dt)).to(DEV)
    v = torch.from_numpy(oracle.ar1((B, Hk, S, D), 0.95, seed + 1)).to(torch_dtype(dt)).to(DEV)
    ks, vs = _CodecStream(fc.make_codec(**cfg)), _CodecStream(fc.make_codec(**cfg))
    if feed == "bulk":
        ks.append(k)
        vs.append(v)
    else:
        for t in range(0, S, feed):
            ks.append(k[..., t:t + feed, :])
            vs.append(v[..., t:t + feed, :])
    return ks, vs


CASES = [
    # name, cfg, dtype, B, Hk, G, S, D
    ("jpeg-i8-f16-g4", dict(mode="jpeg", block_size=8, keep_freqs=4, quant_bits=8), "f16", 2, 4, 4, 8 * 200 + 5, 128),
    ("jpeg-i8-bf16-g8", dict(mode="jpeg", block_size=8, keep_freqs=4, quant_bits=8), "bf16", 1, 2, 8, 8 * 100 + 7, 64),
    ("jpeg-i8-f32-g1", dict(mode="jpeg", block_size=8, keep_freqs=2, quant_bits=8), "f32", 2, 3, 1, 8 * 50 + 3, 32),
    ("jpeg-fp-f32-k8-g2", dict(mode="jpeg", block_size=8, keep_freqs=8), "f32", 1, 2, 2, 8 * 64, 128),
    ("jpeg-fp-f16-k16-g3", dict(mode="jpeg", block_size=16, keep_freqs=16), "f16", 1, 2, 3, 16 * 20 + 9, 64),
    ("jpeg-fp-bf16-g16", dict(mode="jpeg", block_size=8, keep_freqs=2), "bf16", 1, 1, 16, 8 * 40 + 1, 128),
    ("png-f32-k1-g4", dict(mode="png", block_size=8, keep_ratio=1.0), "f32", 2, 2, 4, 8 * 30 + 6, 128),
    ("png-bf16-k05-g2", dict(mode="png", block_size=16, keep_ratio=0.5), "bf16", 1, 2, 2, 16 * 25 + 11, 64),
    ("png-f16-r4-g5", dict(mode="png", block_size=4, keep_ratio=1.0), "f16", 2, 1, 5, 4 * 40 + 2, 16),
    ("png-bf16-r16-k025-g4", dict(mode="png", block_size=16, keep_ratio=0.25), "bf16", 2, 2, 4, 16 * 70 + 9, 128),
    ("png-f16-r8-g3", dict(mode="png", block_size=8, keep_ratio=1.0), "f16", 1, 2, 3, 8 * 90 + 5, 128),
    ("jpeg-i8-f16-d256", dict(mode="jpeg", block_size=8, keep_freqs=4, quant_bits=8), "f16", 1, 2, 4, 8 * 64 + 4, 256),
    ("jpeg-i8-bf16-d512", dict(mode="jpeg", block_size=8, keep_freqs=2, quant_bits=8), "bf16", 1, 1, 2, 8 * 16 + 2, 512),
    ("jpeg-i8-f16-tail-only", dict(mode="jpeg", block_size=8, keep_freqs=4, quant_bits=8), "f16", 2, 2, 4, 5, 128),
    ("jpeg-i8-f32-no-tail", dict(mode="jpeg", block_size=8, keep_freqs=4, quant_bits=8), "f32", 1, 2, 4, 8 * 33, 64),
    ("jpeg-i8-f16-32k", dict(mode="jpeg", block_size=8, keep_freqs=4, quant_bits=8), "f16", 1, 2, 4, 8 * 4096 + 5, 128),
    ("jpeg-i8-f32-r16-d40", dict(mode="jpeg", block_size=16, keep_freqs=3, quant_bits=8), "f32", 1, 2, 2, 16 * 9 + 4, 40),
    ("jpeg-i8-k3-f16-g4", dict(mode="jpeg", block_size=8, keep_freqs=3, quant_bits=8), "f16", 2, 2, 4, 8 * 200 + 5, 128),
    ("jpeg-i8-k8-bf16-g2", dict(mode="jpeg", block_size=8, keep_freqs=8, quant_bits=8), "bf16", 1, 2, 2, 8 * 150 + 3, 128),
    ("jpeg-i8-k3-bf16-d256-g8", dict(mode="jpeg", block_size=8, keep_freqs=3, quant_bits=8), "bf16", 1, 2, 8, 8 * 60 + 7, 256),
    ("jpeg-i8-k8-f16-d64-g16", dict(mode="jpeg", block_size=8, keep_freqs=8, quant_bits=8), "f16", 1, 1, 16, 8 * 70 + 1, 64),
    ("jpeg-i8-r16-k3-f16-g4", dict(mode="jpeg", block_size=16, keep_freqs=3, quant_bits=8), "f16", 1, 2, 4, 16 * 50 + 9, 128),
    ("jpeg-i8-r16-k8-bf16-g1", dict(mode="jpeg", block_size=16, keep_freqs=8, quant_bits=8), "bf16", 2, 2, 1, 16 * 40 + 2, 128),
    ("jpeg-i8-f16-d80-g4", dict(mode="jpeg", block_size=8, keep_freqs=4, quant_bits=8), "f16", 1, 2, 4, 8 * 100 + 3, 80),
    ("jpeg-i8-bf16-d96-g2", dict(mode="jpeg", block_size=8, keep_freqs=2, quant_bits=8), "bf16", 2, 2, 2, 8 * 120 + 5, 96),
    ("jpeg-i8-k3-f16-d96-g8", dict(mode="jpeg", block_size=8, keep_freqs=3, quant_bits=8), "f16", 1, 1, 8, 8 * 90, 96),
    ("jpeg-i8-k8-bf16-d80-g16", dict(mode="jpeg", block_size=8, keep_freqs=8, quant_bits=8), "bf16", 1, 2, 16, 8 * 40 + 7, 80),
    ("png-f32-r16-d128-g4", dict(mode="png", block_size=16, keep_ratio=0.25), "f32", 2, 2, 4, 16 * 100 + 9, 128),
    ("png-f32-r8-d64-g8", dict(mode="png", block_size=8, keep_ratio=1.0), "f32", 1, 2, 8, 8 * 150 + 3, 64),
    ("png-f32-r4-d128-g1", dict(mode="png", block_size=4, keep_ratio=1.0), "f32", 2, 2, 1, 4 * 200 + 1, 128),
    ("png-f32-r16-d64-g16", dict(mode="png", block_size=16, keep_ratio=0.5), "f32", 1, 1, 16, 16 * 40, 64),
    ("png-f32-r8-d128-g5", dict(mode="png", block_size=8, keep_ratio=1.0), "f32", 1, 2, 5, 8 * 80 + 7, 128),
    ("jpeg-i8g-f16-g4", dict(mode="jpeg", block_size=8, keep_freqs=4, quant_bits=8, quant_group=32), "f16", 2, 4, 4, 8 * 200 + 5, 128),
    ("jpeg-i8g-bf16-g2-d64", dict(mode="jpeg", block_size=8, keep_freqs=2, quant_bits=8, quant_group=32), "bf16", 1, 2, 2, 8 * 90 + 3, 64),
    ("jpeg-i8g-f32-r16-d96", dict(mode="jpeg", block_size=16, keep_freqs=3, quant_bits=8, quant_group=32), "f32", 1, 2, 3, 16 * 30 + 9, 96),
    ("jpeg-i8g-f16-d256", dict(mode="jpeg", block_size=8, keep_freqs=4, quant_bits=8, quant_group=32), "f16", 1, 1, 8, 8 * 64 + 1, 256),
    # per-32 scales on the matrix-core pass: rows per block, head groups, widths
    ("i8g-f16-c3", dict(mode="jpeg", block_size=8, keep_freqs=4, quant_bits=8, quant_group=32), "f16", 2, 4, 4, 8 * 400 + 5, 128),
    ("i8g-f16-k8-g16", dict(mode="jpeg", block_size=8, keep_freqs=8, quant_bits=8, quant_group=32), "f16", 1, 1, 16, 8 * 150 + 2, 128),
    ("i8g-bf16-k1-d64-g1", dict(mode="jpeg", block_size=8, keep_freqs=1, quant_bits=8, quant_group=32), "bf16", 2, 2, 1, 8 * 100 + 7, 64),
    ("i8g-bf16-k3-r16-g4", dict(mode="jpeg", block_size=16, keep_freqs=3, quant_bits=8, quant_group=32), "bf16", 1, 2, 4, 16 * 60 + 5, 128),
    ("i8g-bf16-k2-d256-g2", dict(mode="jpeg", block_size=8, keep_freqs=2, quant_bits=8, quant_group=32), "bf16", 1, 2, 2, 8 * 100 + 3, 256),
    ("i8g-f16-k4-d96-g4", dict(mode="jpeg", block_size=8, keep_freqs=4, quant_bits=8, quant_group=32), "f16", 2, 2, 4, 8 * 150 + 6, 96),
    # fp32 queries on per-32 archives: fp32 value products on the matrix cores
    ("i8g-f32-k4-g4", dict(mode="jpeg", block_size=8, keep_freqs=4, quant_bits=8, quant_group=32), "f32", 2, 2, 4, 8 * 300 + 5, 128),
    ("i8g-f32-k8-d64-g16", dict(mode="jpeg", block_size=8, keep_freqs=8, quant_bits=8, quant_group=32), "f32", 1, 1, 16, 8 * 90 + 2, 64),
    ("i8g-f32-k2-d256-g2", dict(mode="jpeg", block_size=8, keep_freqs=2, quant_bits=8, quant_group=32), "f32", 1, 2, 2, 8 * 70 + 3, 256),
    ("i8g-f32-k1-g1", dict(mode="jpeg", block_size=8, keep_freqs=1, quant_bits=8, quant_group=32), "f32", 2, 2, 1, 8 * 120, 128),
    ("i8g-f32-k3-r16-d96-g8", dict(mode="jpeg", block_size=16, keep_freqs=3, quant_bits=8, quant_group=32), "f32", 1, 2, 8, 16 * 50 + 11, 96),
    ("i8g-bf16-k8-r16-d96-g2", dict(mode="jpeg", block_size=16, keep_freqs=8, quant_bits=8, quant_group=32), "bf16", 1, 2, 2, 16 * 70 + 1, 96),
]


I8 = dict(mode="jpeg", block_size=8, keep_freqs=4, quant_bits=8)
CASES += [
    # matrix-core split pass shapes: head groups, rows per block, widths
    ("i8-f16-g16", I8, "f16", 1, 2, 16, 8 * 300 + 3, 128),
    ("i8-bf16-g32", I8, "bf16", 1, 1, 32, 8 * 90 + 6, 128),
    ("i8-f16-g3", I8, "f16", 2, 2, 3, 8 * 77 + 1, 128),
    ("i8-f16-s1", dict(mode="jpeg", block_size=8, keep_freqs=1, quant_bits=8), "f16", 1, 2, 4, 8 * 150 + 2, 128),
    ("i8-bf16-s2-r16", dict(mode="jpeg", block_size=16, keep_freqs=2, quant_bits=8), "bf16", 1, 2, 8, 16 * 70 + 9, 64),
    ("i8-f16-d256-g2", I8, "f16", 1, 2, 2, 8 * 128 + 7, 256),
    ("i8-f16-d64-g4", I8, "f16", 2, 4, 4, 8 * 123 + 4, 64),
    # fp32 queries on the matrix-core pass (four query digits, fp64 logits,
    # two weight halves): head groups, rows per block, widths, tails
    ("i8-f32-c3", I8, "f32", 2, 4, 4, 8 * 400 + 5, 128),
    ("i8-f32-d256-g2", I8, "f32", 1, 2, 2, 8 * 128 + 7, 256),
    ("i8-f32-d64-g8", I8, "f32", 1, 2, 8, 8 * 200 + 3, 64),
    ("i8-f32-s2-r16-g16", dict(mode="jpeg", block_size=16, keep_freqs=2, quant_bits=8), "f32", 1, 1, 16, 16 * 70 + 9, 64),
    ("i8-f32-k8-g1", dict(mode="jpeg", block_size=8, keep_freqs=8, quant_bits=8), "f32", 2, 2, 1, 8 * 150, 128),
    ("i8-f32-k3-d96-g3", dict(mode="jpeg", block_size=8, keep_freqs=3, quant_bits=8), "f32", 1, 2, 3, 8 * 99 + 2, 96),
    ("i8-f32-s1-d80", dict(mode="jpeg", block_size=8, keep_freqs=1, quant_bits=8), "f32", 1, 3, 2, 8 * 180 + 7, 80),
]

P16 = dict(mode="png", block_size=16, keep_ratio=0.25)
CASES += [
    # png and unquantised jpeg stores: head groups of 1-16 (and partial
    # ones), rows per block 1-16, tails, no tail, anchors in every dtype
    ("fp-png-f32-r16-g4", P16, "f32", 2, 2, 4, 16 * 130 + 7, 128),
    ("fp-png-bf16-r16-g8", P16, "bf16", 1, 2, 8, 16 * 64 + 3, 64),
    ("fp-png-f16-r8-g16", dict(mode="png", block_size=8, keep_ratio=1.0), "f16", 1, 1, 16, 8 * 80 + 1, 128),
    ("fp-png-f32-r4-g1", dict(mode="png", block_size=4, keep_ratio=0.5), "f32", 2, 3, 1, 4 * 90, 64),
    ("fp-png-f32-tail-only", P16, "f32", 1, 2, 4, 11, 128),
    ("fp-jpeg-f16-k3-g3", dict(mode="jpeg", block_size=8, keep_freqs=3), "f16", 2, 2, 3, 8 * 111 + 5, 128),
    ("fp-jpeg-f32-k1-g2", dict(mode="jpeg", block_size=8, keep_freqs=1), "f32", 1, 4, 2, 8 * 300 + 2, 64),
    ("fp-jpeg-bf16-k16-g4", dict(mode="jpeg", block_size=16, keep_freqs=16), "bf16", 1, 2, 4, 16 * 33 + 15, 128),
    ("fp-jpeg-f32-k2-g5", dict(mode="jpeg", block_size=8, keep_freqs=2), "f32", 1, 2, 5, 8 * 1000 + 3, 128),
]

FPJ = dict(mode="jpeg", block_size=8, keep_freqs=4)
CASES += [
    # fp16 / bf16 coefficient rows on the matrix-core pass (queries in the
    # stream dtype): rows per block, head groups, widths, tails
    ("fpj-f16-k4-g4", FPJ, "f16", 2, 4, 4, 8 * 300 + 5, 128),
    ("fpj-bf16-k4-g2", FPJ, "bf16", 2, 2, 2, 8 * 260 + 3, 128),
    ("fpj-bf16-k2-d64-g8", dict(FPJ, keep_freqs=2), "bf16", 1, 2, 8, 8 * 200 + 7, 64),
    ("fpj-f16-k8-r16-g16", dict(FPJ, block_size=16, keep_freqs=8), "f16", 1, 2, 16, 16 * 90 + 11, 128),
    ("fpj-bf16-k1-g1", dict(FPJ, keep_freqs=1), "bf16", 2, 3, 1, 8 * 400 + 2, 128),
    ("fpj-f16-k3-d64-g3", dict(FPJ, keep_freqs=3), "f16", 1, 2, 3, 8 * 150 + 1, 64),
    ("fpj-bf16-k4-no-tail", FPJ, "bf16", 1, 2, 4, 8 * 100, 128),
    ("fpj-f16-k2-r4-g5", dict(FPJ, block_size=4, keep_freqs=2), "f16", 1, 2, 5, 4 * 300 + 3, 64),
]


@pytest.fixture
def attention_pass():
    """use(name) selects the split pass for this test ("auto": matrix cores
    for int8 jpeg, fp16 / bf16 jpeg and fp32 png; "valu": the vector-ALU
    pass, the only one for the other stores);
    the previous selection is restored afterwards."""
    from flashcodec_amd import _native as N
    prev = []

    def use(name):
        prev.append(N.set_attention_pass(name))
    yield use
    if prev:
        N.set_attention_pass(prev[0])


@pytest.fixture(params=["auto", "valu"])
def split_variant(request, attention_pass):
    """Run int8 cases on the matrix-core split pass (auto) and on the
    vector-ALU one."""
    attention_pass(request.param)
    return request.param


# int8 cases on both split passes, fp-store cases on their one pass
ORACLE_CASES = [(c, "auto") for c in CASES] + [(c, "valu") for c in CASES
                                                if c[1].get("quant_bits") or c[0].startswith("fpj")]


@pytest.mark.parametrize("case,variant", ORACLE_CASES,
                         ids=[f"{v}-{c[0]}" for c, v in ORACLE_CASES])
def test_decode_attention_matches_oracle(case, variant, oracle, attention_pass):
    name, cfg, dt, B, Hk, G, S, D = case
    attention_pass(variant)
    print(f"case attention/{name} [{variant}]", flush=True)
    seed = seed_of(name)
    ks, vs = build_streams(cfg, dt, B, Hk, S, D, seed % 10000, oracle)
    rng = np.random.default_rng(seed)
    q = torch.from_numpy((rng.standard_normal((B, Hk * G, 1, D)) / math.sqrt(D))
                         .astype(np.float32)).to(torch_dtype(dt)).to(DEV)
    out = fc.codec_decode_attention(q, ks, vs)
    assert out.shape == q.shape and out.dtype == q.dtype
    assert ks._rec is None and vs._rec is None
    ref = oracle_out(oracle, q, ks, vs, D ** -0.5)
    assert_close(to_values(out)[:, :, 0], ref, dt)


@pytest.mark.parametrize("group", [0, 32], ids=["per-row", "per-32"])
@pytest.mark.parametrize("variant", ["auto", "valu"])
def test_fp32_queries_with_sharp_logits(group, variant, oracle, attention_pass):
    """fp32 queries whose logits reach the tens (a nearly one-hot softmax,
    where a logit's rounding moves the output most) on int8 archives with
    one scale per row or per 32 features: within 1e-5 of the fp64 oracle
    on both passes."""
    cfg = dict(mode="jpeg", block_size=8, keep_freqs=4, quant_bits=8, quant_group=group)
    attention_pass(variant)
    B, Hk, G, S, D = 2, 2, 4, 8 * 200 + 3, 128
    print(f"case fp32 sharp logits group={group} [{variant}]", flush=True)
    ks, vs = build_streams(cfg, "f32", B, Hk, S, D, 77, oracle)
    rng = np.random.default_rng(78)
    q = torch.from_numpy((6 * rng.standard_normal((B, Hk * G, 1, D))).astype(np.float32)).to(DEV)
    out = fc.codec_decode_attention(q, ks, vs)
    ref = oracle_out(oracle, q, ks, vs, D ** -0.5)
    assert_close(to_values(out)[:, :, 0], ref, "f32")


@pytest.mark.parametrize("name", Golden("attention").names())
def test_decode_attention_matches_reference_torch_path(name, oracle):
    G = Golden("attention")
    c, m = G.case(name), G.meta[name]
    dt = m["dtype"]
    print(f"case attention-golden/{name}", flush=True)
    k, v, q = to_torch(c["k"], dt), to_torch(c["v"], dt), to_torch(c["q"], dt)
    ks, vs = _CodecStream(fc.make_codec(**m["cfg"])), _CodecStream(fc.make_codec(**m["cfg"]))
    ks.append(k)
    vs.append(v)
    out = to_values(fc.codec_decode_attention(q, ks, vs))[:, :, 0]
    ref_torch = oracle.values_of(c["out"], dt)[:, :, 0]
    ref = oracle_out(oracle, q, ks, vs, m["D"] ** -0.5)
    assert_close(out, ref, dt)
    # and the reference's own path, whose half-precision einsums carry more error
    tol = 1e-5 if dt == "f32" else 4e-3 * np.abs(ref_torch).max()
    assert np.abs(out - ref_torch).max() <= tol


MODES = [("jpeg", dict(keep_freqs=2)), ("jpeg", dict(keep_freqs=8)),
         ("jpeg", dict(keep_freqs=2, quant_bits=8)), ("png", dict(keep_ratio=1.0)),
         ("png", dict(keep_ratio=0.5))]


def test_matches_materialized_attention():
    """Coefficient path == softmax(q K^T) V on the reconstructed view (fp32),
    the reference's tests/test_attention.py:43-53."""
    torch.manual_seed(0)
    B, Hk, S, D = 2, 4, 96, 32
    k_seq = torch.cumsum(torch.randn(B, Hk, S, D, device=DEV) * 0.1, dim=-2)
    v_seq = torch.cumsum(torch.randn(B, Hk, S, D, device=DEV) * 0.1, dim=-2)
    for g in (1, 2):
        q = torch.randn(B, Hk * g, 1, D, device=DEV)
        for mode, kw in MODES:
            cache = fc.CodecKVCache(mode=mode, block_size=8, **kw)
            cache.forward(k_seq, v_seq)
            out = fc.codec_decode_attention(q, cache._keys[0], cache._values[0])
            kr = cache.key_cache[0].repeat_interleave(g, dim=1)
            vr = cache.value_cache[0].repeat_interleave(g, dim=1)
            p = torch.softmax(q @ kr.transpose(-2, -1) / math.sqrt(D), dim=-1)
            ref = p @ vr
            assert (out - ref).abs().max().item() < 1e-5, (mode, kw, g)


def test_no_materialization_and_stream_untouched():
    torch.manual_seed(0)
    cfg = dict(mode="jpeg", block_size=8, keep_freqs=2, quant_bits=8)
    ks, vs = _CodecStream(fc.make_codec(**cfg)), _CodecStream(fc.make_codec(**cfg))
    ks.append(torch.randn(2, 4, 99, 32, device=DEV))
    vs.append(torch.randn(2, 4, 99, 32, device=DEV))
    before = [t.clone() for t in ks._archive_tensors()]
    n, L = ks.n_blocks, ks.seq_len
    out = fc.codec_decode_attention(torch.randn(2, 4, 1, 32, device=DEV), ks, vs)
    assert ks._rec is None and vs._rec is None
    assert ks.n_blocks == n and ks.seq_len == L
    assert all(torch.equal(a, b) for a, b in zip(ks._archive_tensors(), before))
    assert torch.isfinite(out).all()


def test_empty_cache_prefill_guard_and_layouts(oracle):
    cfg = dict(mode="jpeg", block_size=8, keep_freqs=2)
    ks, vs = _CodecStream(fc.make_codec(**cfg)), _CodecStream(fc.make_codec(**cfg))
    q = torch.randn(2, 4, 1, 32, device=DEV)
    assert torch.equal(fc.codec_decode_attention(q, ks, vs), torch.zeros_like(q))
    ks.append(torch.randn(2, 4, 40, 32, device=DEV))
    vs.append(torch.randn(2, 4, 40, 32, device=DEV))
    with pytest.raises(ValueError):
        fc.codec_decode_attention(torch.randn(2, 4, 4, 32, device=DEV), ks, vs)
    # a strided query view (every other head of a wider buffer) and a query
    # dtype other than the stream's
    qt = torch.randn(2, 16, 1, 32, device=DEV)[:, ::2]
    assert not qt.is_contiguous() and qt.stride(-1) == 1
    ref = fc.codec_decode_attention(qt.contiguous(), ks, vs)
    assert torch.equal(fc.codec_decode_attention(qt, ks, vs), ref)
    q16 = qt.to(torch.float16)
    o16 = fc.codec_decode_attention(q16, ks, vs)
    assert o16.dtype == torch.float16
    ref16 = oracle_out(oracle, q16, ks, vs, 32 ** -0.5)
    assert_close(to_values(o16)[:, :, 0], ref16, "f16")


def test_incremental_decode_tracks_oracle(oracle):
    """Token-by-token appends with an attention call after each step (raw tail
    lengths 0..7 and every archive boundary)."""
    cfg = dict(mode="jpeg", block_size=8, keep_freqs=4, quant_bits=8)
    B, Hk, G, D, S = 1, 2, 4, 64, 8 * 5
    ks, vs = _CodecStream(fc.make_codec(**cfg)), _CodecStream(fc.make_codec(**cfg))
    k = torch.from_numpy(oracle.ar1((B, Hk, S, D), 0.9, 5)).half().to(DEV)
    v = torch.from_numpy(oracle.ar1((B, Hk, S, D), 0.9, 6)).half().to(DEV)
    rng = np.random.default_rng(9)
    for t in range(S):
        ks.append(k[..., t:t + 1, :])
        vs.append(v[..., t:t + 1, :])
        q = torch.from_numpy(rng.standard_normal((B, Hk * G, 1, D)).astype(np.float32)
                             / 8).half().to(DEV)
        out = fc.codec_decode_attention(q, ks, vs)
        assert_close(to_values(out)[:, :, 0], oracle_out(oracle, q, ks, vs, D ** -0.5), "f16")


@pytest.mark.parametrize("n_splits", [1, 2, 3, 7, 64, 256])
def test_split_counts_agree(n_splits, oracle, split_variant):
    """Any split count (1 = one workgroup walks 1024 blocks, several passes
    per wavefront; 256 = a few blocks per split) gives the same attention."""
    print(f"case attention/splits={n_splits} [{split_variant}]", flush=True)
    cfg = dict(mode="jpeg", block_size=8, keep_freqs=4, quant_bits=8)
    B, Hk, G, D, S = 2, 2, 4, 128, 8 * 1024 + 3
    ks, vs = build_streams(cfg, "f16", B, Hk, S, D, 77, oracle)
    rng = np.random.default_rng(78)
    q = torch.from_numpy((rng.standard_normal((B, Hk * G, 1, D)) / math.sqrt(D))
                         .astype(np.float32)).half().to(DEV)
    out = fc.codec_decode_attention(q, ks, vs, _n_splits=n_splits)
    assert_close(to_values(out)[:, :, 0], oracle_out(oracle, q, ks, vs, D ** -0.5), "f16")


def _archive_of(st):
    return [t[:, :, :st.n_blocks] for t in st._archive_tensors()] if st.n_blocks else []


I8 = dict(mode="jpeg", block_size=8, keep_freqs=4, quant_bits=8)
# cfg, dtype, D, G, whether the step is one launch (the in-kernel archive)
STEP_PAIRS = [
    (I8, "f16", 64, 4, True),
    (dict(I8, keep_freqs=2), "bf16", 64, 4, True),
    # fp32 coefficient rows (fp32 model, default codec): one launch on the png pass
    (dict(mode="jpeg", block_size=8, keep_freqs=2), "f32", 64, 4, True),
    (dict(mode="jpeg", block_size=16, keep_freqs=4), "f32", 128, 2, True),
    (dict(mode="jpeg", block_size=4, keep_freqs=1), "f32", 128, 8, True),
    (dict(mode="jpeg", block_size=16, keep_freqs=16), "f32", 64, 20, True),
    # fp16 / bf16 coefficient rows: the one-launch step archives them in-kernel
    (dict(mode="jpeg", block_size=8, keep_freqs=4), "bf16", 128, 2, True),
    (dict(mode="jpeg", block_size=8, keep_freqs=2), "f16", 64, 4, True),
    (dict(mode="jpeg", block_size=16, keep_freqs=8), "bf16", 128, 8, True),
    (dict(mode="jpeg", block_size=4, keep_freqs=3), "f16", 128, 1, True),
    # fp32 png: one launch that archives the block (anchor, Top-M deltas) in-kernel
    (dict(mode="png", block_size=8, keep_ratio=0.5), "f32", 64, 4, True),
    (dict(mode="png", block_size=4, keep_ratio=1.0), "f32", 128, 2, True),
    (dict(mode="png", block_size=16, keep_ratio=0.25), "f32", 128, 8, True),
    (dict(mode="png", block_size=8, keep_ratio=0.3), "f32", 64, 16, True),
    # fp16 / bf16 png (16-bit anchors and tails, fp32 deltas): the same launch
    (dict(mode="png", block_size=16, keep_ratio=0.25), "bf16", 128, 4, True),
    (dict(mode="png", block_size=8, keep_ratio=0.5), "f16", 128, 2, True),
    (dict(mode="png", block_size=16, keep_ratio=1.0), "f16", 64, 8, True),
    (dict(mode="png", block_size=4, keep_ratio=1.0), "bf16", 64, 4, True),
    # the C5 instantiation (D=128, bf16, k=4, G=2), other row counts and widths
    (I8, "bf16", 128, 2, True),
    (dict(I8, keep_freqs=3), "f16", 128, 4, True),
    (dict(I8, keep_freqs=8), "bf16", 128, 2, True),
    (I8, "bf16", 80, 4, True),
    (dict(I8, keep_freqs=8), "f16", 96, 4, True),
    (dict(I8, keep_freqs=1), "f16", 256, 8, True),
    (dict(I8, block_size=16, keep_freqs=4), "bf16", 128, 2, True),
    # per-32 scales: the one-launch step archives them in-kernel
    (dict(I8, quant_group=32), "bf16", 128, 2, True),
    (dict(I8, quant_group=32, keep_freqs=8), "f16", 96, 4, True),
    (dict(I8, quant_group=32, keep_freqs=2), "bf16", 64, 1, True),
    (dict(I8, quant_group=32, keep_freqs=1), "f16", 256, 8, True),
    (dict(I8, quant_group=32, block_size=16, keep_freqs=3), "bf16", 128, 16, True),
    # packed Top-M png: one launch that archives the packed block in-kernel
    (dict(mode="png", block_size=8, keep_ratio=0.5, packed=True), "f32", 64, 4, True),
    (dict(mode="png", block_size=16, keep_ratio=0.25, packed=True), "bf16", 128, 4, True),
    (dict(mode="png", block_size=4, keep_ratio=0.67, packed=True), "f16", 256, 16, True),
    (dict(mode="png", block_size=8, keep_ratio=0.75, packed=True), "f32", 128, 2, True),
    # more than 16 query heads per kv head: two head groups, one of them stores
    (I8, "f16", 128, 20, True),
    (dict(mode="png", block_size=8, keep_ratio=0.5), "f32", 64, 20, True),
    (dict(mode="png", block_size=8, keep_ratio=0.5, packed=True), "bf16", 64, 24, True),
    # fp32 queries and stream (an fp32 model): one launch, fp32 rows archived
    # in-kernel
    (I8, "f32", 128, 2, True),
    (dict(I8, keep_freqs=3), "f32", 64, 4, True),
    (dict(I8, quant_group=32), "f32", 128, 2, True),
    (dict(I8, quant_group=32, block_size=16, keep_freqs=2), "f32", 96, 8, True),
]


@pytest.mark.parametrize("cfg,dt,D,G,single", STEP_PAIRS,
                         ids=[f"{c['mode']}-k{c.get('keep_freqs', 0)}-r{c['block_size']}"
                              f"{'-g32' if c.get('quant_group') else ''}"
                              f"{'-packed' if c.get('packed') else ''}-{dt}-D{D}"
                              for c, dt, D, _, _ in STEP_PAIRS])
def test_fused_decode_step_matches_append_then_attend(cfg, dt, D, G, single, oracle):
    """codec_decode_step (one library call per layer step) leaves the same
    archives (codes and scale bits), tails and counters as two appends, and
    its output matches the oracle on them and codec_decode_attention's
    output (two roundings apart), across block boundaries; int8 steps run as
    one launch that archives in-kernel; the first call on uninitialised
    streams takes the two-call path."""
    from flashcodec_amd import _native as N
    B, Hkv = 2, 2
    Hq, r = Hkv * G, cfg["block_size"]
    tdt = torch_dtype(dt)
    print(f"case fused step {cfg} {dt}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(11)
    mk = lambda: fc.make_codec(**cfg)
    ks_f, vs_f, ks_r, vs_r = _CodecStream(mk()), _CodecStream(mk()), _CodecStream(mk()), \
        _CodecStream(mk())
    for st_pair in ((ks_f, ks_r), (vs_f, vs_r)):
        pre = torch.randn((B, Hkv, 2 * r + 3, D), generator=g, device=DEV).to(tdt)
        for st in st_pair:
            st.append(pre)
    fresh_k, fresh_v = _CodecStream(mk()), _CodecStream(mk())
    for step in range(3 * r + 2):
        # HF-style strided views: (B, 1, H, D) projections transposed to (B, H, 1, D)
        q = torch.randn((B, 1, Hq, D), generator=g, device=DEV).to(tdt).transpose(1, 2)
        k = torch.randn((B, 1, Hkv, D), generator=g, device=DEV).to(tdt).transpose(1, 2)
        v = torch.randn((B, 1, Hkv, D), generator=g, device=DEV).to(tdt).transpose(1, 2)
        out_f = fc.codec_decode_step(q, k, v, ks_f, vs_f)
        assert N.lib().fc_last_step_single_launch() == int(single)
        ks_r.append(k)
        vs_r.append(v)
        out_r = fc.codec_decode_attention(q, ks_r, vs_r)
        for a, b in ((ks_f, ks_r), (vs_f, vs_r)):
            assert a.n_blocks == b.n_blocks and a.seq_len == b.seq_len
            for x, y in zip(_archive_of(a), _archive_of(b)):
                assert torch.equal(x, y)
            assert (a.raw is None) == (b.raw is None)
            if a.raw is not None:
                assert torch.equal(a.raw, b.raw)
        assert_close(to_values(out_f)[:, :, 0], oracle_out(oracle, q, ks_f, vs_f, D ** -0.5), dt)
        assert_close_pair(to_values(out_f), to_values(out_r), dt)
        if step == 0:
            out0 = fc.codec_decode_step(q, k, v, fresh_k, fresh_v)   # two-call path
            assert fresh_k.seq_len == 1 and torch.equal(fresh_k.raw, k)
            ref0 = torch.softmax((q.float() @ k.float().transpose(-1, -2).repeat_interleave(
                G, dim=1)) * D ** -0.5, dim=-1) @ v.float().repeat_interleave(G, dim=1)
            assert_close(to_values(out0), ref0.cpu().numpy(), dt)


@pytest.mark.parametrize("name,cfg,dt,B,Hk,G,S,D", [
    ("jpeg-i8-f16", dict(mode="jpeg", block_size=8, keep_freqs=4, quant_bits=8), "f16", 2, 2, 4, 8 * 300 + 5, 128),
    ("png-f32-r16", dict(mode="png", block_size=16, keep_ratio=0.25), "f32", 2, 2, 4, 16 * 90 + 13, 128),
    ("jpeg-fp-bf16", dict(mode="jpeg", block_size=8, keep_freqs=2), "bf16", 1, 2, 8, 8 * 70 + 7, 64),
    ("png-f16-g3", dict(mode="png", block_size=8, keep_ratio=1.0), "f16", 1, 3, 3, 8 * 40 + 1, 64),
], ids=lambda x: x if isinstance(x, str) else None)
def test_split_then_merge_entry_points(name, cfg, dt, B, Hk, G, S, D, oracle):
    """fc_decode_attention_split followed by fc_decode_attention_merge (the
    partials with the raw tail merged by the separate pass) gives the same
    attention as fc_decode_attention (merge fused into the split pass, the
    tail folded into split 0)."""
    from flashcodec_amd import _native as N
    from flashcodec_amd.attention import _device_A, _view, workspace
    print(f"case split+merge {name}", flush=True)
    ks, vs = build_streams(cfg, dt, B, Hk, S, D, seed_of("split-merge", name), oracle)
    assert ks._n_raw > 0
    rng = np.random.default_rng(seed_of("split-merge-q", name))
    q = torch.from_numpy((rng.standard_normal((B, Hk * G, 1, D)) / math.sqrt(D))
                         .astype(np.float32)).to(torch_dtype(dt)).to(DEV)
    fused = fc.codec_decode_attention(q, ks, vs)
    c, r, nb = ks.codec, ks.block_size, ks.n_blocks
    if c.name == "jpeg":
        kind = N.STORE_JPEG_I8 if c.quantized else N.STORE_JPEG_FP
        s = c.keep_freqs
    else:
        kind, s = N.STORE_PNG, r
    L = N.lib()
    dev = q.device
    ns = L.fc_attention_splits(kind, N.dtype_code(ks.dtype), N.dtype_code(q.dtype), s, nb, B, Hk,
                               G, D, N.num_cus(dev))
    ws = workspace(dev, L.fc_attention_workspace_bytes(B, Hk * G, D, ns))
    A = _device_A(c, r, dev)
    keep = []
    kv, vv = _view(ks, keep), _view(vs, keep)
    out = torch.empty_like(q)
    args = (q.data_ptr(), N.dtype_code(q.dtype), q.stride(0), q.stride(1), B, Hk * G, Hk, D, kind,
            N.dtype_code(ks.dtype), r, s, nb, kv, vv, ks._n_raw, N.ptr(A), D ** -0.5,
            out.data_ptr(), out.stride(0), out.stride(1), N.ptr(ws), ns, N.stream_ptr(dev))
    N.check(L.fc_decode_attention_split(*args), "fc_decode_attention_split")
    N.check(L.fc_decode_attention_merge(*args), "fc_decode_attention_merge")
    ref = oracle_out(oracle, q, ks, vs, D ** -0.5)
    assert_close(to_values(out)[:, :, 0], ref, dt)
    assert_close(to_values(fused)[:, :, 0], ref, dt)
    # the workspace counters are back at zero: a second fused call agrees
    again = fc.codec_decode_attention(q, ks, vs)
    assert_close(to_values(again)[:, :, 0], ref, dt)
