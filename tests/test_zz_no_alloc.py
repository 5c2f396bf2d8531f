"""GPU: fc_decode_attention_noalloc (the decode attention with its workspace
in the library's static per-GPU scratch array) against fc_decode_attention
with a caller's workspace, through the C ABI: bitwise equal under the
static pass order, within the contract's tolerance of the oracle, on two
calls in a row (the second smaller), and the size limit reported."""

import ctypes
import math

import numpy as np
import pytest
import torch

import flashcodec_amd as fc
from flashcodec_amd import _native as N
from flashcodec_amd.attention import _device_A, _store_kind, _view, workspace
from tests.conftest import to_values, torch_dtype
from tests.test_gpu_attention import assert_close, build_streams, oracle_out

pytestmark = pytest.mark.gpu
DEV = "cuda"
I8 = dict(mode="jpeg", block_size=8, keep_freqs=4, quant_bits=8)


def _call(entry, q, ks, vs, n_splits, ws=None):
    """One call of `entry` (fc_decode_attention or its _noalloc variant)
    over the two streams (any store kind); returns the output tensor."""
    B, Hq, _, D = q.shape
    Hkv = ks._archive_tensors()[0].shape[1]
    kind, s = _store_kind(ks.codec)
    keep = []
    kv, vv = _view(ks, keep), _view(vs, keep)
    A = _device_A(ks.codec, ks.block_size, q.device)
    out = torch.empty_like(q)
    args = [q.data_ptr(), N.dtype_code(q.dtype), q.stride(0), q.stride(1), B, Hq, Hkv, D,
            kind, N.dtype_code(ks.dtype), ks.block_size, s,
            ks.n_blocks, ctypes.byref(kv), ctypes.byref(vv), ks._n_raw, A.data_ptr(), D ** -0.5,
            out.data_ptr(), out.stride(0), out.stride(1)]
    if ws is not None:
        args.append(ws.data_ptr())
    args += [n_splits, N.stream_ptr(q.device)]
    N.check(entry(*args), entry.__name__)
    return out


@pytest.fixture
def static_order():
    prev = N.set_attention_pass("static")
    yield
    N.set_attention_pass(prev)


@pytest.mark.parametrize("first,second", [
    # (dtype, B, Hkv, G, D, S): the second call is smaller in every dimension
    (("f16", 4, 8, 4, 128, 8 * 3000 + 5), ("f16", 2, 4, 2, 64, 8 * 500 + 3)),
    (("bf16", 2, 8, 2, 128, 8 * 4096 + 1), ("bf16", 1, 2, 4, 128, 8 * 33 + 7)),
])
def test_noalloc_matches_workspace_entry(first, second, oracle, static_order):
    L = N.lib()
    for i, (dt, B, Hkv, G, D, S) in enumerate((first, second)):
        print(f"case noalloc call {i}: {dt} B={B} Hkv={Hkv} G={G} D={D} S={S}", flush=True)
        ks, vs = build_streams(I8, dt, B, Hkv, S, D, 700 + i, oracle)
        rng = np.random.default_rng(701 + i)
        q = torch.from_numpy((rng.standard_normal((B, Hkv * G, 1, D)) / math.sqrt(D))
                             .astype(np.float32)).to(torch_dtype(dt)).to(DEV)
        n_splits = L.fc_attention_splits(N.STORE_JPEG_I8, N.dtype_code(ks.dtype),
                                         N.dtype_code(q.dtype), 4, ks.n_blocks, B, Hkv, G, D,
                                         N.num_cus(q.device))
        ws = workspace(q.device, L.fc_attention_workspace_bytes(B, Hkv * G, D, n_splits))
        ref_ws = _call(L.fc_decode_attention, q, ks, vs, n_splits, ws)
        got = _call(L.fc_decode_attention_noalloc, q, ks, vs, n_splits)
        torch.cuda.synchronize()
        assert torch.equal(got, ref_ws)
        assert_close(to_values(got)[:, :, 0], oracle_out(oracle, q, ks, vs, D ** -0.5), dt)


@pytest.mark.parametrize("cfg,first,second", [
    # other store kinds through the same entry: png (16-bit anchors), packed
    # Top-M png, fp16 / bf16 / fp32 coefficient jpeg, per-32 int8 jpeg
    (dict(mode="png", block_size=16, keep_ratio=0.25), ("bf16", 2, 8, 4, 128, 16 * 900 + 5),
     ("bf16", 1, 2, 2, 64, 16 * 40 + 3)),
    (dict(mode="png", block_size=8, keep_ratio=0.5, packed=True), ("f32", 2, 4, 4, 128, 8 * 1500),
     ("f32", 1, 2, 2, 64, 8 * 60 + 1)),
    (dict(mode="jpeg", block_size=8, keep_freqs=2), ("bf16", 4, 8, 2, 128, 8 * 2000 + 3),
     ("bf16", 2, 2, 4, 64, 8 * 100 + 1)),
    (dict(I8, quant_group=32), ("f16", 4, 8, 4, 128, 8 * 2000 + 5), ("f16", 1, 2, 2, 96, 8 * 70)),
    (dict(mode="jpeg", block_size=8, keep_freqs=4), ("f32", 2, 8, 4, 128, 8 * 2000 + 3),
     ("f32", 1, 2, 2, 64, 8 * 90 + 1)),
], ids=["png-bf16", "pngpk-f32", "fpj-bf16", "i8g-f16", "fpj-f32"])
def test_noalloc_other_store_kinds(cfg, first, second, oracle, static_order):
    L = N.lib()
    for i, (dt, B, Hkv, G, D, S) in enumerate((first, second)):
        print(f"case noalloc {cfg} call {i}: {dt} B={B} Hkv={Hkv} G={G} D={D} S={S}", flush=True)
        ks, vs = build_streams(cfg, dt, B, Hkv, S, D, 710 + i, oracle)
        rng = np.random.default_rng(711 + i)
        q = torch.from_numpy((rng.standard_normal((B, Hkv * G, 1, D)) / math.sqrt(D))
                             .astype(np.float32)).to(torch_dtype(dt)).to(DEV)
        kind, s = _store_kind(ks.codec)
        n_splits = L.fc_attention_splits(kind, N.dtype_code(ks.dtype), N.dtype_code(q.dtype), s,
                                         ks.n_blocks, B, Hkv, G, D, N.num_cus(q.device))
        ws = workspace(q.device, L.fc_attention_workspace_bytes(B, Hkv * G, D, n_splits))
        ref_ws = _call(L.fc_decode_attention, q, ks, vs, n_splits, ws)
        got = _call(L.fc_decode_attention_noalloc, q, ks, vs, n_splits)
        torch.cuda.synchronize()
        assert torch.equal(got, ref_ws)
        assert_close(to_values(got)[:, :, 0], oracle_out(oracle, q, ks, vs, D ** -0.5), dt)


def test_noalloc_rejects_calls_beyond_its_scratch():
    L = N.lib()
    B, Hq, D, n_splits = 64, 64, 512, 64
    assert L.fc_attention_workspace_bytes(B, Hq, D, n_splits) > N.NOALLOC_SCRATCH_BYTES
    rc = L.fc_decode_attention_noalloc(None, N.F16, 0, 0, B, Hq, 8, D, N.STORE_JPEG_I8, N.F16,
                                       8, 4, 4096, None, None, 0, None, 1.0, None, 0, 0,
                                       n_splits, None)
    assert rc == N.ERR_SCRATCH
    assert b"scratch" in L.fc_status_string(rc)
