"""ctypes binding of ``libflashcodec_amd.so`` (the C ABI of include/flashcodec_amd.h).

The library is loaded after ``import torch`` so that it binds to the HIP
runtime PyTorch already loaded (both carry the soname libamdhip64.so.7).
There is no fallback: if the library is missing or a kernel reports an error
the call raises.
"""

import ctypes
import os

import torch

from . import _build

F32, F16, BF16, I8 = 0, 1, 2, 3
OK, ERR_ARG, ERR_UNSUPPORTED, ERR_HIP, ERR_SCRATCH = 0, -1, -2, -3, -5
NOALLOC_SCRATCH_BYTES = 16 << 20
PASS_AUTO, PASS_VECTOR, PASS_STATIC = 0, 1, 2
STORE_JPEG_I8, STORE_JPEG_FP, STORE_PNG, STORE_JPEG_I8G, STORE_PNG_PACKED = 0, 1, 2, 3, 4
MAX_BLOCK = 64
MAX_HEAD_DIM = 512

_DTYPE_CODE = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16, torch.int8: I8}

_i64 = ctypes.c_int64
_int = ctypes.c_int
_vp = ctypes.c_void_p
_fp = ctypes.c_float


class StreamView(ctypes.Structure):
    """fc_stream_view: one KV stream as seen by the decode attention."""
    _fields_ = [
        ("rows", _vp), ("scales", _vp), ("anchors", _vp), ("cap", _i64),
        ("raw", _vp), ("raw_sb", _i64), ("raw_sh", _i64), ("raw_st", _i64), ("masks", _vp),
    ]


class StepStream(ctypes.Structure):
    """fc_step_stream: one stream of a layer for fc_decode_step."""
    _fields_ = [
        ("rows", _vp), ("scales", _vp), ("anchors", _vp), ("cap", _i64), ("tail", _vp),
        ("token", _vp), ("tok_sb", _i64), ("tok_sh", _i64), ("masks", _vp),
    ]


class StepArgs(ctypes.Structure):
    """fc_step_args: the arguments of fc_decode_step."""
    _fields_ = [
        ("q", _vp), ("q_dtype", _int), ("q_sb", _i64), ("q_sh", _i64),
        ("B", _i64), ("Hq", _i64), ("Hkv", _i64), ("D", _i64),
        ("store_kind", _int), ("stream_dtype", _int), ("r", _int), ("s", _int),
        ("quant_bits", _int), ("keep_m", _int), ("n_blocks", _i64), ("n_tail", _i64),
        ("basis", _vp), ("A", _vp), ("scale", _fp), ("out", _vp), ("o_sb", _i64), ("o_sh", _i64),
        ("workspace", _vp), ("workspace_bytes", _i64), ("n_cu", _int), ("stream", _vp),
        ("key", StepStream), ("value", StepStream), ("state", _vp),
    ]


_ATTN_SIG = (_int, [_vp, _int, _i64, _i64, _i64, _i64, _i64, _i64, _int, _int, _int, _int, _i64,
                    ctypes.POINTER(StreamView), ctypes.POINTER(StreamView), _i64, _vp, _fp, _vp,
                    _i64, _i64, _vp, _int, _vp])

# name -> (restype, argtypes)
SIGNATURES = {
    "fc_version": (_int, []),
    "fc_status_string": (ctypes.c_char_p, [_int]),
    "fc_last_hip_error": (_int, []),
    "fc_jpeg_encode": (_int, [_vp, _int, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                              _int, _int, _vp, _vp, _vp, _i64, _i64, _int, _vp]),
    "fc_jpeg_decode": (_int, [_vp, _int, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _int, _int,
                              _vp, _vp, _int, _i64, _i64, _i64, _i64, _vp]),
    "fc_jpeg_encode_grouped": (_int, [_vp, _int, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                                      _int, _int, _vp, _vp, _vp, _i64, _i64, _int, _vp]),
    "fc_jpeg_decode_grouped": (_int, [_vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _int, _int,
                                      _int, _vp, _vp, _int, _i64, _i64, _i64, _i64, _vp]),
    "fc_quantize_rows": (_int, [_vp, _int, _i64, _i64, _i64, _vp, _vp, _vp]),
    "fc_dequantize_rows": (_int, [_vp, _vp, _i64, _i64, _vp, _int, _vp]),
    "fc_png_encode": (_int, [_vp, _int, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _int,
                             _int, _vp, _vp, _i64, _i64, _vp]),
    "fc_png_decode": (_int, [_vp, _vp, _int, _i64, _i64, _i64, _i64, _i64, _i64, _int, _vp,
                             _i64, _i64, _i64, _i64, _vp]),
    "fc_png_encode_packed": (_int, [_vp, _int, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                                    _int, _int, _vp, _vp, _vp, _i64, _i64, _vp]),
    "fc_png_decode_packed": (_int, [_vp, _vp, _vp, _int, _i64, _i64, _i64, _i64, _i64, _i64,
                                    _int, _int, _vp, _i64, _i64, _i64, _i64, _vp]),
    "fc_png_unpack": (_int, [_vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _int, _int, _vp,
                             _i64, _vp]),
    "fc_attention_workspace_bytes": (_i64, [_i64, _i64, _i64, _int]),
    "fc_attention_default_splits": (_int, [_i64, _i64, _i64, _i64, _int]),
    "fc_attention_splits": (_int, [_int, _int, _int, _int, _i64, _i64, _i64, _i64, _i64, _int]),
    "fc_decode_attention": _ATTN_SIG,
    "fc_decode_attention_split": _ATTN_SIG,
    "fc_decode_attention_merge": _ATTN_SIG,
    "fc_png_topm_mask_host": (ctypes.c_uint64, [_vp, _int, _int]),
    "fc_decode_step": (_int, [ctypes.POINTER(StepArgs)]),
    "fc_last_step_single_launch": (_int, []),
    "fc_prefill_attention": (_int, [_vp, _int, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                                    _i64, _int, _int, _int, _int, _i64, ctypes.POINTER(StreamView),
                                    ctypes.POINTER(StreamView), _i64, _vp, _fp, _vp, _i64, _i64,
                                    _i64, _vp]),
    "fc_gather_segments": (_int, [_vp, _i64, _i64, _vp, _i64, _i64, _vp, _i64, _i64, _i64, _i64,
                                  _vp]),
    "fc_decode_attention_noalloc": (_int, _ATTN_SIG[1][:21] + [_int, _vp]),
    "fc_set_attention_pass": (_int, [_int]),
    "fc_get_attention_pass": (_int, []),
}

_LIB = None


def library_path():
    return _build.LIB_PATH


def lib():
    """The loaded library (raises if it has not been built)."""
    global _LIB
    if _LIB is None:
        path = library_path()
        if not os.path.exists(path):
            raise RuntimeError(
                f"flashcodec_amd native library not found at {path}; build it with "
                "`python -m flashcodec_amd._build` (or __graft_entry__.build())")
        handle = ctypes.CDLL(path)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = handle
    return _LIB


class KernelError(RuntimeError):
    """A flashcodec_amd kernel entry point returned an error status."""


def check(rc, what):
    if rc == OK:
        return
    L = lib()
    msg = L.fc_status_string(rc).decode()
    if rc == ERR_HIP:
        msg += f" (hipError {L.fc_last_hip_error()})"
    if rc == ERR_UNSUPPORTED:
        raise NotImplementedError(f"{what}: {msg}")
    raise KernelError(f"{what}: {msg}")


def set_attention_pass(name):
    """Select the decode-attention split pass process-wide: "auto" (matrix
    cores for the int8 jpeg archives they support, passes from a queue),
    "static" (the same with a fixed pass order: bitwise reproducible) or
    "valu" (vector ALU for every store, for A/B measurements).  Returns the
    previous name."""
    names = {PASS_AUTO: "auto", PASS_VECTOR: "valu", PASS_STATIC: "static"}
    L = lib()
    prev = names[L.fc_get_attention_pass()]
    code = {v: k for k, v in names.items()}[name]
    check(L.fc_set_attention_pass(code), "fc_set_attention_pass")
    return prev


def dtype_code(dtype):
    try:
        return _DTYPE_CODE[dtype]
    except KeyError:
        raise TypeError(f"unsupported dtype {dtype} (expected float32, float16, bfloat16"
                        " or int8)") from None


def require_gpu(*tensors):
    """Every tensor must live on a ROCm device: this package has no CPU path."""
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise RuntimeError(
                "flashcodec_amd computes on the GPU only (HIP kernels for gfx950); "
                f"got a tensor on {t.device}. Move the KV tensors to a ROCm device.")


_RAW_STREAM = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_ptr(device):
    """hipStream_t of torch's current stream on `device`."""
    if _RAW_STREAM is not None:
        idx = device.index if device.index is not None else torch.cuda.current_device()
        return _RAW_STREAM(idx)
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t):
    return None if t is None else t.data_ptr()


_N_CU = {}


def num_cus(device):
    idx = device.index if device.index is not None else torch.cuda.current_device()
    if idx not in _N_CU:
        _N_CU[idx] = torch.cuda.get_device_properties(idx).multi_processor_count
    return _N_CU[idx]
