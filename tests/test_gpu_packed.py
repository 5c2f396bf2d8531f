"""GPU: the packed Top-M png archive (PNGCodec(packed=True)): archive bits
against the oracle's packing of png_filter's output, unpacking and
reconstruction bit for bit against the dense archive, decode attention on
the packed pass against the fp64 oracle (and the dense archive's), the
decode-step paths and the structural operations.

png_filter / png_reconstruct follow flashcodec/codecs/png.py:36-74; the
packed layout is this build's (the reference leaves Top-M sparsity unpacked,
README.md:580-583).  Tolerances as test_gpu_attention (fp32: 1e-5 absolute;
fp16 / bf16: 2e-3 of max|ref| plus half an ulp).
"""

import math

import numpy as np
import pytest
import torch

import flashcodec_amd as fc
from flashcodec_amd import _native as N
from flashcodec_amd.cache import _CodecStream
from tests.conftest import bits, to_values, torch_dtype
from tests.test_gpu_attention import assert_close, build_streams, oracle_out

pytestmark = pytest.mark.gpu
DEV = "cuda"


def packed(r, keep):
    return dict(mode="png", block_size=r, keep_ratio=keep, packed=True)


def dense(r, keep):
    return dict(mode="png", block_size=r, keep_ratio=keep)


def tokens(oracle, dt, shape, seed):
    return torch.from_numpy(oracle.ar1(shape, 0.97, seed)).to(torch_dtype(dt)).to(DEV)


ARCHIVE_CASES = [(16, 0.25, "f32"), (16, 0.5, "bf16"), (8, 0.5, "f16"), (4, 0.5, "f32"),
                 (8, 0.25, "bf16"), (16, 0.1, "f32"), (12, 0.3, "f32"), (2, 0.5, "f32")]


@pytest.mark.parametrize("r,keep,dt", ARCHIVE_CASES)
@pytest.mark.parametrize("feed", ["bulk", 1, 5])
def test_packed_archive_bits_match_oracle(r, keep, dt, feed, oracle):
    """Values, mask words and anchors of a packed stream (bulk, token-by-token
    and chunked appends) equal the oracle's packing of png_filter's output
    bit for bit; unpacking them on the device gives png_filter's dense deltas
    bit for bit (the dense archive's own bits, -0.0 included)."""
    B, H, D = 2, 3, 64
    S = r * 37 + (r // 2)
    print(f"case packed archive r={r} keep={keep} {dt} feed={feed}", flush=True)
    x = tokens(oracle, dt, (B, H, S, D), 11 + r)
    st = _CodecStream(fc.make_codec(**packed(r, keep)))
    ref = _CodecStream(fc.make_codec(**dense(r, keep)))
    for s_ in (st, ref):
        if feed == "bulk":
            s_.append(x)
        else:
            for t in range(0, S, feed):
                s_.append(x[:, :, t:t + feed])
    n = st.n_blocks
    assert n == S // r and ref.n_blocks == n
    xv = to_values(x)[:, :, :n * r]
    d, a = oracle.png_encode(xv, r, keep)
    keep_m = oracle.png_keep_m(r, keep)
    vals, mask = oracle.png_pack(d, keep_m)
    assert np.array_equal(bits(st._packed[:, :, :n].cpu().numpy()), bits(vals))
    assert np.array_equal(st._packed_mask[:, :, :n].cpu().numpy().view(np.uint32), mask)
    assert torch.equal(st._anchors[:, :, :n], ref._anchors[:, :, :n])
    un = fc.codecs.png_unpack(st._packed[:, :, :n], st._packed_mask[:, :, :n], r)
    assert torch.equal(un.view(torch.int32), ref._deltas[:, :, :n].contiguous().view(torch.int32))
    assert np.array_equal(bits(un.cpu().numpy()), bits(d))


@pytest.mark.parametrize("r,keep,dt", ARCHIVE_CASES[:5])
def test_packed_read_matches_dense_read(r, keep, dt, oracle):
    """read() of a packed stream is the dense archive's reconstruction bit
    for bit (png_reconstruct: fp64 running sum), raw tail included, and so
    is a crop that cuts into the archive."""
    B, H, D = 2, 2, 128
    S = r * 25 + r // 2 + 1
    x = tokens(oracle, dt, (B, H, S, D), 21 + r)
    st = _CodecStream(fc.make_codec(**packed(r, keep)))
    ref = _CodecStream(fc.make_codec(**dense(r, keep)))
    st.append(x)
    ref.append(x)
    assert torch.equal(st.read(), ref.read())
    d, a = oracle.png_encode(to_values(x)[:, :, :st.n_blocks * r], r, keep)
    rec = oracle.png_decode(d, a, dt)
    assert np.array_equal(to_values(st.read())[:, :, :st.n_blocks * r], rec)
    for s_ in (st, ref):
        s_.crop(-(r + 3))
    assert st.seq_len == ref.seq_len and st.n_blocks == ref.n_blocks
    assert torch.equal(st.read(), ref.read())


# name, r, keep, dtype, B, Hkv, G, S, D
ATTN_CASES = [
    ("r16-k025-f32-g4", 16, 0.25, "f32", 2, 2, 4, 16 * 90 + 7, 128),
    ("r16-k05-bf16-g2", 16, 0.5, "bf16", 1, 2, 2, 16 * 60 + 11, 128),
    ("r8-k05-f16-g8", 8, 0.5, "f16", 2, 1, 8, 8 * 120 + 3, 64),
    ("r4-k05-f32-g1", 4, 0.5, "f32", 1, 3, 1, 4 * 200 + 1, 128),
    ("r16-k01-f32-g16", 16, 0.1, "f32", 1, 1, 16, 16 * 40 + 2, 64),
    ("r12-k03-f32-g3", 12, 0.3, "f32", 2, 2, 3, 12 * 50 + 5, 256),
    ("r8-k025-bf16-g5", 8, 0.25, "bf16", 1, 2, 5, 8 * 70, 128),
    ("r16-k025-f32-g32", 16, 0.25, "f32", 1, 1, 32, 16 * 30 + 9, 64),
    ("r16-k05-f16-d256-g4", 16, 0.5, "f16", 1, 2, 4, 16 * 33 + 15, 256),
    ("r6-k04-f32-tail-only", 6, 0.4, "f32", 2, 2, 4, 5, 128),
    ("r16-k025-f32-g4-large", 16, 0.25, "f32", 2, 4, 4, 16 * 2000, 128),
]


@pytest.mark.parametrize("case", ATTN_CASES, ids=[c[0] for c in ATTN_CASES])
def test_packed_attention_matches_oracle(case, oracle):
    """Decode attention on the packed pass against the fp64 oracle on the
    unpacked rows, and against the dense archive's attention (same rows)."""
    name, r, keep, dt, B, Hkv, G, S, D = case
    print(f"case packed attention {name}", flush=True)
    ks, vs = build_streams(packed(r, keep), dt, B, Hkv, S, D, 31 + r + D, oracle)
    dk, dv = build_streams(dense(r, keep), dt, B, Hkv, S, D, 31 + r + D, oracle)
    rng = np.random.default_rng(32)
    q = torch.from_numpy((rng.standard_normal((B, Hkv * G, 1, D)) / math.sqrt(D))
                         .astype(np.float32)).to(torch_dtype(dt)).to(DEV)
    out = fc.codec_decode_attention(q, ks, vs)
    assert out.dtype == q.dtype and out.shape == q.shape
    ref = oracle_out(oracle, q, ks, vs, D ** -0.5)
    assert_close(to_values(out)[:, :, 0], ref, dt)
    assert_close(to_values(fc.codec_decode_attention(q, dk, dv))[:, :, 0], ref, dt)


@pytest.mark.parametrize("n_splits", [1, 3, 7, 64])
def test_packed_split_counts_and_two_pass_entry(n_splits, oracle):
    """Any split count gives the oracle's attention; the split pass with the
    merge as its own launch (fc_decode_attention_split + _merge) too."""
    from flashcodec_amd.attention import _device_A, _view, workspace
    B, Hkv, G, D, r = 2, 2, 4, 128, 16
    S = r * 700 + 9
    ks, vs = build_streams(packed(r, 0.25), "f32", B, Hkv, S, D, 41, oracle)
    rng = np.random.default_rng(42)
    q = torch.from_numpy((rng.standard_normal((B, Hkv * G, 1, D)) / math.sqrt(D))
                         .astype(np.float32)).to(DEV)
    ref = oracle_out(oracle, q, ks, vs, D ** -0.5)
    out = fc.codec_decode_attention(q, ks, vs, _n_splits=n_splits)
    assert_close(to_values(out)[:, :, 0], ref, "f32")
    L = N.lib()
    nb = ks.n_blocks
    per = -(-nb // n_splits)
    ns = -(-nb // per)
    dev = q.device
    ws = workspace(dev, L.fc_attention_workspace_bytes(B, Hkv * G, D, ns))
    keep = []
    kv, vv = _view(ks, keep), _view(vs, keep)
    A = _device_A(ks.codec, r, dev)
    out2 = torch.empty_like(q)
    args = (q.data_ptr(), N.F32, q.stride(0), q.stride(1), B, Hkv * G, Hkv, D,
            N.STORE_PNG_PACKED, N.F32, r, ks.codec.keep_m, nb, kv, vv, ks._n_raw, N.ptr(A),
            D ** -0.5, out2.data_ptr(), out2.stride(0), out2.stride(1), N.ptr(ws), ns,
            N.stream_ptr(dev))
    N.check(L.fc_decode_attention_split(*args), "fc_decode_attention_split")
    N.check(L.fc_decode_attention_merge(*args), "fc_decode_attention_merge")
    assert_close(to_values(out2)[:, :, 0], ref, "f32")


@pytest.mark.parametrize("keep", [0.25, 0.5])
def test_c4_packed_full_shape(keep, oracle):
    """BASELINE C4's shape on packed archives: fp32 (2, 8, 16384, 128),
    r=16, 32 q heads, fp32 queries; the archive is (2 + keep_m) / 16 of the
    dense one's bytes."""
    B, Hkv, G, D, S, r = 2, 8, 4, 128, 16384, 16
    print(f"case c4 packed keep={keep}", flush=True)
    ks, vs = build_streams(packed(r, keep), "f32", B, Hkv, S, D, 404, oracle)
    m = ks.codec.keep_m
    assert ks.storage_bytes() == B * Hkv * (S // r) * D * 4 * (2 + m)
    rng = np.random.default_rng(405)
    q = torch.from_numpy((rng.standard_normal((B, Hkv * G, 1, D)) / math.sqrt(D))
                         .astype(np.float32)).to(DEV)
    out = fc.codec_decode_attention(q, ks, vs)
    assert_close(to_values(out)[:, :, 0], oracle_out(oracle, q, ks, vs, D ** -0.5), "f32")


def test_packed_structural_ops(oracle):
    """Capacity growth, beam reorders (in place), batch selection and crops
    keep packed archives equal to a dense twin's unpacked bits and the same
    attention."""
    B, Hkv, G, D, r = 3, 2, 2, 64, 8
    x = [tokens(oracle, "f32", (B, Hkv, r * 20 + 3, D), s) for s in (51, 52)]
    ks, vs = _CodecStream(fc.make_codec(**packed(r, 0.5))), \
        _CodecStream(fc.make_codec(**packed(r, 0.5)))
    dk, dv = _CodecStream(fc.make_codec(**dense(r, 0.5))), \
        _CodecStream(fc.make_codec(**dense(r, 0.5)))
    for t in range(0, x[0].shape[2], 7):                      # grows 16 -> 32 blocks
        for st, xx in ((ks, x[0]), (vs, x[1]), (dk, x[0]), (dv, x[1])):
            st.append(xx[:, :, t:t + 7])
    idx = torch.tensor([2, 0, 0], device=DEV)
    for st in (ks, vs, dk, dv):
        st.select_batch(idx)
        st.crop(-5)
    for p_, d_ in ((ks, dk), (vs, dv)):
        n = p_.n_blocks
        un = fc.codecs.png_unpack(p_._packed[:, :, :n], p_._packed_mask[:, :, :n], r)
        assert torch.equal(un.view(torch.int32), d_._deltas[:, :, :n].contiguous().view(torch.int32))
        assert torch.equal(p_.read(), d_.read())
    q = torch.randn((B, Hkv * G, 1, D), device=DEV) / 8
    ref = oracle_out(oracle, q, ks, vs, D ** -0.5)
    assert_close(to_values(fc.codec_decode_attention(q, ks, vs))[:, :, 0], ref, "f32")
    for st in (ks, vs):
        st.select_batch(torch.tensor([1], device=DEV))       # batch selection (out of place)
    q1 = q[1:2]
    assert_close(to_values(fc.codec_decode_attention(q1, ks, vs))[:, :, 0],
                 oracle_out(oracle, q1, ks, vs, D ** -0.5), "f32")


def test_packed_codec_arguments():
    """Packing is a png option with keep_ratio < 1 and at most 8 kept deltas;
    the storage ratio counts the anchor, the kept deltas and the mask word."""
    with pytest.raises(ValueError):
        fc.make_codec("jpeg", packed=True)
    with pytest.raises(ValueError):
        fc.make_codec("png", block_size=32, keep_ratio=0.1, packed=True)
    with pytest.raises(ValueError):
        fc.make_codec("png", block_size=16, keep_ratio=0.75, packed=True)
    c = fc.make_codec("png", block_size=16, keep_ratio=0.25, packed=True)
    assert c.keep_m == 4 and c.storage_ratio() == 6 / 16
