"""CPU: the C-ABI library loads, exports everything include/flashcodec_amd.h
declares, validates arguments before touching a device, and its host-side
Top-M selection matches the oracle (torch's CPU topk order)."""

import ctypes
import os
import re
import shutil
import subprocess

import numpy as np
import pytest

from flashcodec_amd import _native as N

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "flashcodec_amd.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(fc_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(N.library_path())
    names = declared_functions()
    assert len(names) >= 12
    for name in names:
        assert hasattr(lib, name), name
    # the Python binding declares exactly the header's functions
    assert sorted(N.SIGNATURES) == names


def test_version_and_status_strings():
    L = N.lib()
    assert L.fc_version() == 100
    assert L.fc_status_string(0) == b"ok"
    assert b"invalid" in L.fc_status_string(N.ERR_ARG)


def test_workspace_and_split_policy():
    L = N.lib()
    assert L.fc_attention_workspace_bytes(8, 32, 128, 32) >= 8 * 32 * 32 * 130 * 4
    assert L.fc_attention_workspace_bytes(8, 32, 128, 0) == 0
    assert L.fc_attention_default_splits(0, 8, 8, 4, 256) == 0
    for nb in (1, 7, 63, 4096, 100000):
        for cols in ((1, 1, 1), (8, 8, 4), (16, 8, 2), (1, 32, 1)):
            ns = L.fc_attention_default_splits(nb, *cols, 256)
            assert 1 <= ns <= 256
            bps = -(-nb // ns)
            assert bps * (ns - 1) < nb          # no empty split


def test_store_aware_split_count():
    """int8 jpeg stores with half-precision queries take the matrix-core
    split count (at most one round, at least one pass per wavefront, at most
    max(16, passes / 10)); other stores one round of the vector-ALU pass (two
    workgroups per compute unit when no device reports the occupancy)."""
    L = N.lib()
    assert L.fc_attention_splits(N.STORE_PNG, N.F32, N.F32, 16, 0, 2, 8, 4, 128, 256) == 0
    # the measured shapes: C3, C5, and the reference's published ones
    assert L.fc_attention_splits(N.STORE_JPEG_I8, N.F16, N.F16, 4, 4096, 8, 8, 4, 128, 256) == 8
    assert L.fc_attention_splits(N.STORE_JPEG_I8, N.F16, N.F16, 4, 512, 16, 8, 2, 128, 256) == 4
    assert L.fc_attention_splits(N.STORE_JPEG_I8, N.F16, N.F16, 2, 2048, 1, 8, 2, 128, 256) == 16
    assert L.fc_attention_splits(N.STORE_JPEG_I8, N.F16, N.F16, 2, 8192, 1, 8, 2, 128, 256) == 25
    for nb in (1, 7, 1024, 4096, 100000):
        for cols in ((8, 8, 4), (2, 8, 4), (1, 32, 1)):
            ns = L.fc_attention_splits(N.STORE_JPEG_I8, N.F16, N.F16, 4, nb, *cols, 128, 256)
            assert 1 <= ns <= L.fc_attention_default_splits(nb, *cols, 256)
            passes = -(-nb * 4 // 64)
            assert ns <= max(1, passes // 4)
            assert -(-nb // ns) * (ns - 1) < nb       # no empty split
            for kind, s in ((N.STORE_PNG, 16), (N.STORE_JPEG_FP, 2), (N.STORE_JPEG_I8, 4)):
                ns = L.fc_attention_splits(kind, N.F32, N.F32, s, nb, *cols, 128, 256)
                assert 1 <= ns <= 256
                assert -(-nb // ns) * (ns - 1) < nb   # no empty split


def test_argument_validation_needs_no_device():
    L = N.lib()
    # k > r, bad quant bits, store overflow, bad dtype: rejected up front
    assert L.fc_jpeg_encode(None, 0, 1, 1, 0, 0, 0, 8, 1, 16, 8, 9, None, None, None, 1, 0, 0,
                            None) == N.ERR_ARG
    assert L.fc_jpeg_encode(None, 0, 1, 1, 0, 0, 0, 8, 1, 16, 8, 2, None, None, None, 1, 0, 4,
                            None) == N.ERR_ARG
    assert L.fc_jpeg_encode(None, 0, 1, 1, 0, 0, 0, 8, 2, 16, 8, 2, None, None, None, 1, 0, 0,
                            None) == N.ERR_ARG
    assert L.fc_png_encode(None, 9, 1, 1, 0, 0, 0, 8, 1, 16, 8, 0, None, None, 1, 0,
                           None) == N.ERR_ARG
    assert L.fc_jpeg_decode(None, 0, None, 1, 1, 4, 3, 2, 16, 8, 2, None, None, 0, 0, 0, 0, 0,
                            None) == N.ERR_ARG
    # nothing to do is fine without pointers
    assert L.fc_jpeg_encode(None, 0, 0, 1, 0, 0, 0, 8, 1, 16, 8, 2, None, None, None, 1, 0, 0,
                            None) == N.OK
    # attention: Hq not a multiple of Hkv, empty cache
    kv = N.StreamView()
    assert L.fc_decode_attention(1, 0, 0, 0, 1, 3, 2, 16, 0, 0, 8, 2, 1, kv, kv, 0, None, 1.0,
                                 1, 0, 0, None, 1, None) == N.ERR_ARG
    assert L.fc_decode_attention(1, 0, 0, 0, 1, 2, 2, 16, 0, 0, 8, 2, 0, kv, kv, 0, None, 1.0,
                                 1, 0, 0, None, 1, None) == N.ERR_ARG
    # beyond the kernels' limits
    assert L.fc_jpeg_encode(1, 0, 1, 1, 0, 0, 0, 128, 1, 16, 128, 2, 1, 1, None, 1, 0, 0,
                            None) == N.ERR_UNSUPPORTED


def _topm_host(col, m):
    L = N.lib()
    v = np.ascontiguousarray(col, np.float32)
    mask = L.fc_png_topm_mask_host(v.ctypes.data_as(ctypes.c_void_p), v.shape[0], m)
    return np.array([(mask >> i) & 1 for i in range(v.shape[0])], bool)


@pytest.mark.parametrize("n", [1, 3, 7, 15, 31, 63])
def test_host_topm_matches_oracle_under_ties(oracle, n):
    rng = np.random.default_rng(n)
    for m in sorted({1, 2, max(1, n // 4), max(1, n // 2), max(1, n - 1)}):
        for trial in range(150):
            kind = trial % 4
            if kind == 0:
                v = rng.integers(-2, 3, n).astype(np.float32)
            elif kind == 1:
                v = (rng.integers(-5, 6, n) * 0.25).astype(np.float32)
            elif kind == 2:
                v = rng.standard_normal(n).astype(np.float32)
            else:
                v = rng.integers(-1, 2, n).astype(np.float32)
                v[rng.integers(0, n, 2)] = np.nan
            got = _topm_host(v, m)
            want = oracle.topk_keep(np.abs(v), min(m, n))
            assert np.array_equal(got, want), (n, m, v)


def test_host_topm_adversarial_orders(oracle):
    """Sorted, reversed and organ-pipe columns drive introselect's pivots to
    extremes (the heap-selection fallback included)."""
    for n in (15, 31, 63):
        base = np.arange(n, dtype=np.float32)
        cols = [base, base[::-1].copy(), np.concatenate([base[::2], base[1::2][::-1]]),
                np.minimum(base, base[::-1]), np.full(n, 3.0, np.float32),
                (base % 3).astype(np.float32), (base // 4).astype(np.float32)]
        for v in cols:
            for m in range(1, n):
                assert np.array_equal(_topm_host(v, m), oracle.topk_keep(np.abs(v), m)), (n, m)


@pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc not available")
def test_struct_layouts_match_the_header(tmp_path):
    """The ctypes mirrors of fc_stream_view, fc_step_stream and fc_step_args
    have the C compiler's field offsets and sizes."""
    structs = {"fc_stream_view": N.StreamView, "fc_step_stream": N.StepStream,
               "fc_step_args": N.StepArgs}
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "flashcodec_amd.h"',
             'int main(void) {']
    for cname, py in structs.items():
        lines.append(f'  printf("{cname} size %zu\\n", sizeof({cname}));')
        for field, _ in py._fields_:
            lines.append(f'  printf("{cname} {field} %zu\\n", offsetof({cname}, {field}));')
    lines += ['  return 0;', '}']
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", f"-I{os.path.join(ROOT, 'include')}", str(src), "-o", str(exe)],
                   check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout
    got = {}
    for line in out.splitlines():
        cname, field, val = line.split()
        got[(cname, field)] = int(val)
    for cname, py in structs.items():
        assert got[(cname, "size")] == ctypes.sizeof(py), cname
        for field, _ in py._fields_:
            assert got[(cname, field)] == getattr(py, field).offset, (cname, field)
