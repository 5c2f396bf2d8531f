"""GPU: _CodecStream / CodecKVCache behaviour — golden archive and read()
bits through the real append path, causal safety, memoised reads, exact and
repeatable crops, beam reorders, storage accounting (the behaviours of the
reference's tests/test_causal.py)."""

import math

import numpy as np
import pytest
import torch

import flashcodec_amd as fc
from flashcodec_amd.cache import _CodecStream
from tests.conftest import Golden, bits, to_torch, to_values

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _archive(st):
    if st.codec.name == "jpeg":
        out = [st._coeffs[:, :, :st.n_blocks]]
        if st.codec.quantized:
            out.append(st._scales[:, :, :st.n_blocks])
        return out
    return [st._deltas[:, :, :st.n_blocks], st._anchors[:, :, :st.n_blocks]]


@pytest.mark.parametrize("name", Golden("stream").names())
def test_stream_matches_reference_bits(name, oracle):
    G = Golden("stream")
    c, m = G.case(name), G.meta[name]
    cfg, dt, feed = m["cfg"], m["dtype"], m["feed"]
    print(f"case stream/{name}", flush=True)
    x = to_torch(c["x"], dt)
    st = _CodecStream(fc.make_codec(**cfg))
    S = x.shape[-2]
    if feed == "bulk":
        st.append(x)
    else:
        step = 1 if feed == "token" else int(feed)
        for t in range(0, S, step):
            st.append(x[..., t:t + step, :])
    assert st.n_blocks == m["n_blocks"] and st.seq_len == S
    if cfg["mode"] == "jpeg":
        got = to_values(st._coeffs[:, :, :st.n_blocks])
        want = c["coeffs"].astype(np.float32) if cfg.get("quant_bits") else \
            oracle.values_of(c["coeffs"], dt)
        assert np.array_equal(bits(got), bits(want))
        if cfg.get("quant_bits"):
            assert np.array_equal(bits(st._scales[:, :, :st.n_blocks, :, 0].cpu().numpy()),
                                  bits(c["scales"]))
    else:
        assert np.array_equal(bits(st._deltas[:, :, :st.n_blocks].cpu().numpy()),
                              bits(c["deltas"]))
        assert np.array_equal(bits(to_values(st._anchors[:, :, :st.n_blocks])),
                              bits(oracle.values_of(c["anchors"], dt)))
    assert np.array_equal(bits(to_values(st.read())), bits(oracle.values_of(c["read"], dt)))
    st.crop(-5)
    assert np.array_equal(bits(to_values(st.read())),
                          bits(oracle.values_of(c["read_crop5"], dt)))


B, H, S, D, R = 2, 4, 96, 32, 8


@pytest.fixture(scope="module")
def seqs():
    torch.manual_seed(0)
    return (torch.randn(B, H, S, D, device=DEV), torch.randn(B, H, S, D, device=DEV))


def _fill_incr(k_seq, v_seq, **cfg):
    cache = fc.CodecKVCache(**cfg)
    for t in range(k_seq.shape[-2]):
        cache.decode_step(k_seq[..., t:t + 1, :], v_seq[..., t:t + 1, :])
    return cache


def toy_attn(q, k, v):
    Sq, Sk = q.shape[-2], k.shape[-2]
    logits = q @ k.transpose(-2, -1) / math.sqrt(q.shape[-1])
    mask = torch.ones(Sq, Sk, dtype=torch.bool, device=q.device).tril(diagonal=Sk - Sq)
    return torch.softmax(logits.masked_fill(~mask, float("-inf")), dim=-1) @ v


def test_future_perturbation_never_rewrites_archive(seqs):
    k_seq, v_seq = seqs
    c = fc.CodecKVCache(mode="png", block_size=R, keep_ratio=0.5)
    cut = 2 * R
    for t in range(cut):
        c.decode_step(k_seq[..., t:t + 1, :], v_seq[..., t:t + 1, :])
    snap = [[t.clone() for t in _archive(st)] for st in (c._keys[0], c._values[0])]
    view = c.key_cache[0].clone()
    pert = torch.randn_like(k_seq[..., cut:, :])
    for t in range(S - cut):
        c.decode_step(pert[..., t:t + 1, :], pert[..., t:t + 1, :])
    for st, sn in zip((c._keys[0], c._values[0]), snap):
        for now, before in zip(_archive(st), sn):
            assert torch.equal(now[:, :, :before.shape[2]], before)
    assert torch.equal(c.key_cache[0][..., :cut, :], view[..., :cut, :])
    # full-sequence fill: perturbing tokens after a block boundary leaves the
    # earlier blocks' coefficients and view untouched
    c1 = fc.CodecKVCache(mode="jpeg", block_size=R, keep_freqs=2)
    c2 = fc.CodecKVCache(mode="jpeg", block_size=R, keep_freqs=2)
    k2 = k_seq.clone()
    k2[..., 3 * R:, :] = torch.randn_like(k2[..., 3 * R:, :])
    c1.forward(k_seq, v_seq)
    c2.forward(k2, v_seq)
    assert torch.equal(c1._keys[0]._coeffs[:, :, :3], c2._keys[0]._coeffs[:, :, :3])
    assert torch.equal(c1.key_cache[0][..., :3 * R, :], c2.key_cache[0][..., :3 * R, :])


def test_incremental_matches_full_on_lossless_png(seqs):
    k_seq, v_seq = seqs
    q = torch.randn(B, H, S, D, device=DEV)
    c_full = fc.CodecKVCache(mode="png", block_size=R, keep_ratio=1.0)
    kf, vf = c_full.forward(k_seq, v_seq)
    out_full = toy_attn(q, kf, vf)
    c = fc.CodecKVCache(mode="png", block_size=R, keep_ratio=1.0)
    outs = []
    for t in range(S):
        kt, vt = c.decode_step(k_seq[..., t:t + 1, :], v_seq[..., t:t + 1, :])
        outs.append(toy_attn(q[..., t:t + 1, :], kt, vt))
    assert (out_full - torch.cat(outs, dim=-2)).abs().max() < 1e-4


@pytest.mark.parametrize("mode,kw", [("jpeg", dict(keep_freqs=2)), ("png", dict(keep_ratio=1.0)),
                                     ("jpeg", dict(keep_freqs=4, quant_bits=8))])
def test_memoised_read_equals_fresh_fill_bitwise(seqs, mode, kw):
    """Blocks are encoded and decoded independently of how they were batched,
    so incremental and one-shot fills agree bit for bit."""
    k_seq, v_seq = seqs
    c = fc.CodecKVCache(mode=mode, block_size=R, **kw)
    for t in range(S):
        c.decode_step(k_seq[..., t:t + 1, :], v_seq[..., t:t + 1, :])
        if t % 13 == 0 or t == S - 1:
            fresh = fc.CodecKVCache(mode=mode, block_size=R, **kw)
            fresh.forward(k_seq[..., :t + 1, :], v_seq[..., :t + 1, :])
            assert torch.equal(c.key_cache[0], fresh.key_cache[0])
            assert torch.equal(c.value_cache[0], fresh.value_cache[0])


@pytest.mark.parametrize("mode,kw", [("png", dict(keep_ratio=1.0)), ("jpeg", dict(keep_freqs=2))])
def test_crop_exact_and_repeatable(seqs, mode, kw):
    k_seq, v_seq = seqs
    c = _fill_incr(k_seq, v_seq, mode=mode, block_size=R, **kw)
    k_ref, v_ref = c.key_cache[0].clone(), c.value_cache[0].clone()
    c.crop(-5)
    assert c.get_seq_length(0) == S - 5
    assert torch.equal(c.key_cache[0], k_ref[..., :-5, :])
    assert torch.equal(c.value_cache[0], v_ref[..., :-5, :])
    c2 = _fill_incr(k_seq, v_seq, mode=mode, block_size=R, **kw)
    c2.crop(-2)
    c2.crop(-3)
    assert torch.equal(c2.key_cache[0], k_ref[..., :-5, :])
    c3 = _fill_incr(k_seq, v_seq, mode=mode, block_size=R, **kw)
    c3.crop(-S)
    assert c3.get_seq_length(0) == 0
    c4 = _fill_incr(k_seq, v_seq, mode=mode, block_size=R, **kw)
    c4.crop(-(S - 3 * R))
    assert torch.equal(c4.key_cache[0], k_ref[..., :3 * R, :])
    # the stream keeps working after a crop
    c.decode_step(k_seq[..., :1, :], v_seq[..., :1, :])
    assert c.get_seq_length(0) == S - 4


@pytest.mark.parametrize("mode,kw", [("png", dict(keep_ratio=1.0)), ("jpeg", dict(keep_freqs=2)),
                                     ("jpeg", dict(keep_freqs=2, quant_bits=8))])
def test_reorder_cache_permutes_archives(mode, kw):
    torch.manual_seed(1)
    b = 4
    kb, vb = torch.randn(b, H, S, D, device=DEV), torch.randn(b, H, S, D, device=DEV)
    idx = torch.tensor([2, 0, 3, 1])
    c = fc.CodecKVCache(mode=mode, block_size=R, **kw)
    k_ref, v_ref = c.forward(kb, vb)
    c.reorder_cache(idx)
    assert torch.equal(c.key_cache[0], k_ref.index_select(0, idx.to(DEV)))
    assert torch.equal(c.value_cache[0], v_ref.index_select(0, idx.to(DEV)))
    c.decode_step(kb.index_select(0, idx.to(DEV))[..., :1, :],
                  vb.index_select(0, idx.to(DEV))[..., :1, :])
    assert c.get_seq_length(0) == S + 1
    # batch-size change (beam expansion)
    c.reorder_cache(torch.tensor([0, 0, 1, 1, 2, 2]))
    assert c.key_cache[0].shape[0] == 6


def test_int8_storage_and_causal_contract(seqs):
    k_seq, v_seq = seqs
    cq = fc.CodecKVCache(mode="jpeg", block_size=R, keep_freqs=2, quant_bits=8)
    kq, vq = cq.forward(k_seq, v_seq)
    ci = _fill_incr(k_seq, v_seq, mode="jpeg", block_size=R, keep_freqs=2, quant_bits=8)
    assert torch.equal(kq, ci.key_cache[0]) and torch.equal(vq, ci.value_cache[0])
    plain = fc.CodecKVCache(mode="jpeg", block_size=R, keep_freqs=2)
    plain.forward(k_seq, v_seq)
    assert cq.storage_bytes(0) < 0.5 * plain.storage_bytes(0)
    # exact accounting: int8 codes + fp32 scales per archived block, K and V
    n = S // R
    assert cq.storage_bytes(0) == 2 * B * H * n * (2 * D + 2 * 4)
    cq.crop(-5)
    cq.reorder_cache(torch.tensor([1, 0]))
    assert cq.get_seq_length(0) == S - 5
    st = cq.stats(0)
    assert st["tokens"] == S - 5 and st["archived"] + st["raw"] == S - 5


def test_capacity_growth_keeps_prefix():
    torch.manual_seed(2)
    st = _CodecStream(fc.make_codec("jpeg", block_size=8, keep_freqs=4, quant_bits=8))
    x = torch.randn(1, 2, 8 * 40, 64, device=DEV, dtype=torch.float16)
    st.append(x[..., :8 * 16, :])
    assert st._capacity == 16
    before = st._coeffs[:, :, :16].clone()
    st.append(x[..., 8 * 16:, :])
    assert st._capacity == 64 and st.n_blocks == 40
    assert torch.equal(st._coeffs[:, :, :16], before)
    one = _CodecStream(fc.make_codec("jpeg", block_size=8, keep_freqs=4, quant_bits=8))
    one.append(x)
    assert torch.equal(one._coeffs[:, :, :40], st._coeffs[:, :, :40])
    assert torch.equal(one.read(), st.read())


@pytest.mark.parametrize("mode,kw", [("jpeg", dict(keep_freqs=4, quant_bits=8)),
                                     ("jpeg", dict(keep_freqs=2)),
                                     ("png", dict(keep_ratio=0.5))])
def test_ragged_appends_keep_the_tail_and_equal_a_bulk_fill(seqs, mode, kw):
    """Appends of mixed sizes (inside the tail, completing it, spanning
    several blocks) leave the last seq_len % r input tokens as the raw tail
    after every call and archive exactly what one bulk append archives."""
    k_seq, _ = seqs
    cfg = dict(mode=mode, block_size=R, **kw)
    print(f"case ragged {mode} {kw}", flush=True)
    bulk = _CodecStream(fc.make_codec(**cfg))
    bulk.append(k_seq)
    st = _CodecStream(fc.make_codec(**cfg))
    sizes = [1, 3, 8, 13, 2, 5, 17, 1, 7, 9, 0, 16, 4]
    pos, i = 0, 0
    while pos < S:
        m = min(sizes[i % len(sizes)], S - pos)
        st.append(k_seq[..., pos:pos + m, :])
        pos, i = pos + m, i + 1
        t = pos % R
        assert st.seq_len == pos and st.n_blocks == pos // R
        if t:
            assert torch.equal(st.raw, k_seq[..., pos - t:pos, :])
        else:
            assert st.raw is None
    for a, b in zip(_archive(st), _archive(bulk)):
        assert torch.equal(a, b)
    assert torch.equal(st.read(), bulk.read())


def test_tail_reads_are_copies_and_follow_batch_changes(seqs):
    k_seq, _ = seqs
    cfg = dict(mode="jpeg", block_size=R, keep_freqs=4, quant_bits=8)
    st = _CodecStream(fc.make_codec(**cfg))
    st.append(k_seq[..., :3, :])
    r0 = st.read()
    st.append(k_seq[..., 3:3 + R, :])          # completes a block, rewrites the tail
    assert torch.equal(r0, k_seq[..., :3, :])
    assert torch.equal(st.raw, k_seq[..., R:R + 3, :])
    idx = torch.tensor([1, 0, 1], device=DEV)  # batch 2 -> 3 with a live tail
    st.select_batch(idx)
    assert torch.equal(st.raw, k_seq[idx][..., R:R + 3, :])
    st.append(k_seq[idx][..., R + 3:2 * R + 1, :])
    ref = _CodecStream(fc.make_codec(**cfg))
    ref.append(k_seq[idx][..., :2 * R + 1, :])
    for a, b in zip(_archive(st), _archive(ref)):
        assert torch.equal(a, b)
    assert torch.equal(st.raw, ref.raw) and torch.equal(st.read(), ref.read())
