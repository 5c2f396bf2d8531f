"""flashcodec_amd — MI355X-native KV-cache codec (drop-in for flashcodec 1.x).

Compresses a transformer KV cache (B, H, S, D) along the token axis:
  mode="jpeg": blockwise orthonormal DCT-II, keep k of r frequencies,
               optionally int8 with one scale per (block, frequency);
  mode="png":  per-block anchor + fp32 first-order deltas, optional Top-M.
Archive, reconstruction and materialisation-free decode attention run as
hand-written HIP kernels for gfx950 behind a C ABI (libflashcodec_amd.so,
include/flashcodec_amd.h).  Public names follow flashcodec/__init__.py:13-37.
"""

from .attention import block_basis, codec_decode_attention, codec_decode_step
from .cache import HAS_HF_CACHE, CodecKVCache, FlashCodecCache, FlashCodecLayer, make_codec
from .codecs import (JPEGCodec, PNGCodec, dct_basis, dct_compress, dct_decompress,
                     dequantize_coeffs, png_filter, png_reconstruct, quantize_coeffs)
from .patch import apply_flash_codec, find_attention_modules, remove_flash_codec, \
    undo_flash_codec
from .patch_attention import apply_codec_attention, codec_attention_stats, \
    remove_codec_attention

__version__ = "1.0.0"

__all__ = [
    "apply_flash_codec", "remove_flash_codec", "undo_flash_codec",
    "find_attention_modules",
    "apply_codec_attention", "remove_codec_attention", "codec_attention_stats",
    "CodecKVCache", "FlashCodecCache", "FlashCodecLayer", "make_codec",
    "HAS_HF_CACHE", "JPEGCodec", "PNGCodec",
    "codec_decode_attention", "block_basis",
    "dct_basis", "dct_compress", "dct_decompress",
    "quantize_coeffs", "dequantize_coeffs",
    "png_filter", "png_reconstruct",
    "__version__",
]
