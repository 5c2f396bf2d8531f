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
    with pytest.raises(ValueError):
        fc.codec_decode_attention(torch.randn(1, 2, 1, 8), ks, vs, impl="torch")
    # empty cache: zeros, no device work
    out = fc.codec_decode_attention(torch.randn(1, 2, 1, 8), ks, vs)
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
