"""CPU: the host-side API surface (names, argument checks and error types
of the reference), and that nothing computes on the CPU."""

import pytest
import torch

import flashcodec_amd as fc
from flashcodec_amd.cache import _CodecStream

REFERENCE_ALL = [
    "apply_flash_codec", "remove_flash_codec", "undo_flash_codec", "find_attention_modules",
    "apply_codec_attention", "remove_codec_attention", "codec_attention_stats",
    "CodecKVCache", "FlashCodecCache", "FlashCodecLayer", "make_codec", "HAS_HF_CACHE",
    "JPEGCodec", "PNGCodec", "codec_decode_attention", "block_basis", "dct_basis",
    "dct_compress", "dct_decompress", "quantize_coeffs", "dequantize_coeffs", "png_filter",
    "png_reconstruct", "__version__",
]


def test_public_names_match_reference():
    assert sorted(fc.__all__) == sorted(REFERENCE_ALL)
    for name in REFERENCE_ALL:
        assert hasattr(fc, name)
    assert fc.__version__ == "1.0.0"
    assert fc.HAS_HF_CACHE


def test_make_codec_errors_and_repr():
    with pytest.raises(ValueError):
        fc.make_codec("png", quant_bits=8)
    with pytest.raises(ValueError):
        fc.make_codec("webp")
    with pytest.raises(AssertionError):
        fc.make_codec("jpeg", block_size=8, keep_freqs=9)
    with pytest.raises(AssertionError):
        fc.make_codec("jpeg", quant_bits=4)
    with pytest.raises(AssertionError):
        fc.make_codec("png", keep_ratio=0.0)
    c = fc.make_codec("jpeg", block_size=8, keep_freqs=2, quant_bits=8)
    assert c.quantized and repr(c) == "JPEGCodec(block_size=8, keep_freqs=2, quant_bits=8)"
    assert abs(c.storage_ratio() - 0.0625) < 1e-12
    assert fc.make_codec("jpeg", keep_freqs=2).storage_ratio() == 0.25
    p = fc.make_codec("png", block_size=16, keep_ratio=0.25)
    assert p.storage_ratio() == 1.0 and p.keep_m == 4
    assert fc.make_codec("png", block_size=16, keep_ratio=1.0).keep_m == 0
    plain = fc.JPEGCodec(block_size=8, keep_freqs=2)
    assert plain.quantize(None) == (None, None)


def test_quantize_rejects_other_bit_widths():
    with pytest.raises(ValueError):
        fc.quantize_coeffs(torch.zeros(1, 2, 4), bits=4)


def test_cpu_tensors_fail_loudly():
    x = torch.randn(1, 2, 16, 8)
    with pytest.raises(RuntimeError, match="GPU"):
        fc.dct_compress(x, 8, 2)
    with pytest.raises(RuntimeError, match="GPU"):
        fc.png_filter(x, 8)
    st = _CodecStream(fc.make_codec("jpeg"))
    with pytest.raises(RuntimeError, match="GPU"):
        st.append(x)


def test_decode_attention_argument_errors():
    ks = _CodecStream(fc.make_codec("jpeg"))
    vs = _CodecStream(fc.make_codec("jpeg"))
    with pytest.raises(ValueError):
        fc.codec_decode_attention(torch.randn(1, 2, 4, 8), ks, vs)       # prefill shape
    # the reference's impl="triton" raises when its Triton path cannot run a
    # jpeg case (here: an empty archive; flashcodec/attention.py:91-99)
    with pytest.raises(RuntimeError, match="triton"):
        fc.codec_decode_attention(torch.randn(1, 2, 1, 8), ks, vs, impl="triton")
    # empty cache: zeros, no device work, whichever implementation is named
    for impl in ("auto", "torch", "hip"):
        out = fc.codec_decode_attention(torch.randn(1, 2, 1, 8), ks, vs, impl=impl)
        assert torch.equal(out, torch.zeros(1, 2, 1, 8))
    # png stores never take the reference's Triton branch: no error there
    ps = _CodecStream(fc.make_codec("png")), _CodecStream(fc.make_codec("png"))
    out = fc.codec_decode_attention(torch.randn(1, 2, 1, 8), *ps, impl="triton")
    assert torch.equal(out, torch.zeros(1, 2, 1, 8))


def test_block_basis_shapes():
    A = fc.block_basis(fc.make_codec("jpeg", block_size=8, keep_freqs=3), 8)
    assert A.shape == (8, 3) and torch.equal(A, fc.dct_basis(8, 3).t())
    T = fc.block_basis(fc.make_codec("png", block_size=4), 4)
    assert torch.equal(T, torch.tril(torch.ones(4, 4)))


def test_stream_empty_state():
    st = _CodecStream(fc.make_codec("png", block_size=8))
    assert st.seq_len == 0 and st.read() is None and st.storage_bytes() == 0
    st.crop(-3)
    assert st.seq_len == 0
    with pytest.raises(ValueError):
        st.crop(2)


def test_graph_host_counters_advance_like_appends():
    """graph.advance_host moves a layer's host counters the way one-token
    appends do: the tail grows to r - 1, then a block moves to the archive."""
    pytest.importorskip("transformers")
    from flashcodec_amd import graph
    from flashcodec_amd.cache import FlashCodecLayer

    class Cache:
        pass

    r = 8
    layer = FlashCodecLayer(mode="jpeg", block_size=r, keep_freqs=4, quant_bits=8)
    cache = Cache()
    cache.layers = [layer, object()]             # non-codec layers are left alone
    for st in (layer._key_stream, layer._value_stream):
        st.n_blocks, st.n_archived, st._n_raw = 3, 3 * r, 5
    seen = []
    for _ in range(13):
        graph.advance_host(cache)
        st = layer._key_stream
        seen.append((st.n_blocks, st._n_raw))
    assert seen[:4] == [(3, 6), (3, 7), (4, 0), (4, 1)]
    assert seen[-1] == (5, 2)                    # 3 blocks + 5 + 13 = 42 tokens = 5 * 8 + 2
    twin = FlashCodecLayer(mode="jpeg", block_size=r, keep_freqs=4, quant_bits=8)
    cache2 = Cache()
    cache2.layers = [twin]
    for st in (twin._key_stream, twin._value_stream):
        st.n_blocks, st.n_archived, st._n_raw = 3, 3 * r, 5
    graph.advance_host(cache2, steps=13)
    for a, b in ((layer._key_stream, twin._key_stream), (layer._value_stream, twin._value_stream)):
        assert (a.n_blocks, a.n_archived, a._n_raw) == (b.n_blocks, b.n_archived, b._n_raw)
        assert a.n_archived == r * a.n_blocks


def test_graph_prepare_refuses_mixed_and_empty_caches():
    pytest.importorskip("transformers")
    from flashcodec_amd import graph
    from flashcodec_amd.cache import FlashCodecLayer

    class Cache:
        pass

    cache = Cache()
    cache.layers = [FlashCodecLayer(mode="jpeg", block_size=8, keep_freqs=4, quant_bits=8),
                    object()]
    with pytest.raises(NotImplementedError):
        graph.prepare(cache, 16)
    cache.layers = [FlashCodecLayer(mode="png", block_size=8)]
    with pytest.raises(ValueError):               # no archived block to size the splits
        graph.prepare(cache, 16)


def test_fused_step_codec_equality():
    """The fused decode step archives both streams with one codec setting:
    equal parameters qualify, any difference does not."""
    from flashcodec_amd.attention import _same_codec
    mk = fc.make_codec
    assert _same_codec(mk(mode="jpeg", block_size=8, keep_freqs=4, quant_bits=8),
                       mk(mode="jpeg", block_size=8, keep_freqs=4, quant_bits=8))
    assert not _same_codec(mk(mode="jpeg", block_size=8, keep_freqs=4, quant_bits=8),
                           mk(mode="jpeg", block_size=8, keep_freqs=4))
    assert not _same_codec(mk(mode="jpeg", block_size=8, keep_freqs=4),
                           mk(mode="jpeg", block_size=8, keep_freqs=2))
    assert _same_codec(mk(mode="png", block_size=16, keep_ratio=0.25),
                       mk(mode="png", block_size=16, keep_ratio=0.25))
    assert not _same_codec(mk(mode="png", block_size=16, keep_ratio=0.25),
                           mk(mode="png", block_size=16, keep_ratio=0.5))
    assert not _same_codec(mk(mode="png", block_size=8), mk(mode="jpeg", block_size=8))


def test_plain_causal_mask_recognition():
    """The attention patch runs a prefill on the archive only under a mask
    the kernel applies (the plain causal one): None, an all-kept 2-D padding
    mask, or the exact causal pattern as a bool or additive float 4-D mask
    (also over a longer key axis); padded or shifted masks are refused."""
    import torch
    from flashcodec_amd.patch_attention import _plain_causal
    T, P0 = 5, 3
    total = P0 + T
    keys = torch.arange(total)
    allowed = keys[None, :] <= torch.arange(P0, total)[:, None]
    bmask = allowed[None, None].expand(2, 1, T, total).clone()
    fmask = torch.where(bmask, 0.0, torch.finfo(torch.float32).min)
    assert _plain_causal(None, T, total)
    assert _plain_causal(torch.ones(2, total, dtype=torch.long), T, total)
    assert _plain_causal(bmask, T, total)
    assert _plain_causal(fmask, T, total)
    longer = torch.cat([fmask, torch.full((2, 1, T, 4), torch.finfo(torch.float32).min)], -1)
    assert _plain_causal(longer, T, total)
    pad2d = torch.ones(2, total, dtype=torch.long)
    pad2d[1, 0] = 0
    assert not _plain_causal(pad2d, T, total)
    padded = bmask.clone()
    padded[1, :, :, :2] = False                   # left padding of sequence 1
    assert not _plain_causal(padded, T, total)
    assert not _plain_causal(torch.where(padded, 0.0, -1e9), T, total)
    full = torch.ones_like(bmask)                 # bidirectional
    assert not _plain_causal(full, T, total)
    assert not _plain_causal(bmask[..., 1:], T, total)   # fewer keys than cached
    assert not _plain_causal(object(), T, total)
