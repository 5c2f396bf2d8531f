"""GPU: seeded random sweeps over the shape space of the png paths (dense
and packed archives) and the jpeg paths (int8 with one scale per row or per
32 features, unquantised coefficients): fp32 / fp16 / bf16 streams, block
sizes, keep ratios / kept frequencies, head sizes, query heads per kv head,
batch, tails; each case against the fp64 oracle on the streams' rows, and
decode steps against two appends.

The cases are drawn once from a fixed seed (the same list on every run), so
a failure names a reproducible configuration.
"""

import math

import numpy as np
import pytest
import torch

import flashcodec_amd as fc
from tests.conftest import to_values, torch_dtype
from tests.test_gpu_attention import (_archive_of, assert_close, assert_close_pair, build_streams,
                                      oracle_out)

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _draw(seed, n, packed):
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        r = int(rng.choice([4, 8, 16]))
        keep = float(rng.choice([0.25, 0.5, 0.75] if packed else [0.25, 0.5, 1.0]))
        if packed and math.ceil((r - 1) * keep) > 8:
            keep = 0.5
        dt = str(rng.choice(["f32", "f16", "bf16"]))
        D = int(rng.choice([64, 128]))
        G = int(rng.choice([1, 2, 3, 4, 6, 8, 16, 20]))
        B = int(rng.integers(1, 4))
        Hkv = int(rng.choice([1, 2, 4]))
        S = int(rng.integers(1, 60)) * r + int(rng.integers(0, r))
        out.append((dict(mode="png", block_size=r, keep_ratio=keep, packed=packed), dt, B, Hkv,
                    G, S, D))
    return out


ATTN = _draw(2024, 24, False) + _draw(2025, 16, True)


@pytest.mark.parametrize("case", ATTN, ids=[f"a{i}" for i in range(len(ATTN))])
def test_png_attention_sweep(case, oracle):
    cfg, dt, B, Hkv, G, S, D = case
    print(f"case png sweep {case}", flush=True)
    ks, vs = build_streams(cfg, dt, B, Hkv, S, D, 900 + S, oracle)
    rng = np.random.default_rng(S + D)
    q = torch.from_numpy((rng.standard_normal((B, Hkv * G, 1, D)) / math.sqrt(D))
                         .astype(np.float32)).to(torch_dtype(dt)).to(DEV)
    out = fc.codec_decode_attention(q, ks, vs)
    assert_close(to_values(out)[:, :, 0], oracle_out(oracle, q, ks, vs, D ** -0.5), dt)


STEPS = _draw(2026, 10, False) + _draw(2027, 8, True)


def _step_sweep(case, oracle):
    """r + 2 fused steps from a random archive state: archives, tails and
    counters equal two appends' bit for bit, outputs within the contract of
    the oracle and of codec_decode_attention after the appends."""
    cfg, dt, B, Hkv, G, S, D = case
    r = cfg["block_size"]
    print(f"case step sweep {case}", flush=True)
    ks_f, vs_f = build_streams(cfg, dt, B, Hkv, S, D, 700 + S, oracle)
    ks_r, vs_r = build_streams(cfg, dt, B, Hkv, S, D, 700 + S, oracle)
    g = torch.Generator(device=DEV).manual_seed(S)
    tdt = torch_dtype(dt)
    for _ in range(r + 2):
        q = torch.randn((B, 1, Hkv * G, D), generator=g, device=DEV).to(tdt).transpose(1, 2)
        k = torch.randn((B, 1, Hkv, D), generator=g, device=DEV).to(tdt).transpose(1, 2)
        v = torch.randn((B, 1, Hkv, D), generator=g, device=DEV).to(tdt).transpose(1, 2)
        out_f = fc.codec_decode_step(q, k, v, ks_f, vs_f)
        ks_r.append(k)
        vs_r.append(v)
        out_r = fc.codec_decode_attention(q, ks_r, vs_r)
        for a, b in ((ks_f, ks_r), (vs_f, vs_r)):
            assert a.n_blocks == b.n_blocks and a.seq_len == b.seq_len
            for x, y in zip(_archive_of(a), _archive_of(b)):
                assert torch.equal(x, y)
            if a.raw is not None:
                assert torch.equal(a.raw, b.raw)
        assert_close(to_values(out_f)[:, :, 0], oracle_out(oracle, q, ks_f, vs_f, D ** -0.5), dt)
        assert_close_pair(to_values(out_f), to_values(out_r), dt)


@pytest.mark.parametrize("case", STEPS, ids=[f"s{i}" for i in range(len(STEPS))])
def test_png_step_sweep(case, oracle):
    _step_sweep(case, oracle)


def _draw_jpeg(seed, n):
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        r = int(rng.choice([4, 8, 16]))
        k = int(rng.integers(1, min(r, 8) + 1))
        quant = int(rng.choice([8, 8, 0]))
        dt = str(rng.choice(["f32", "f16", "bf16"]))
        D = int(rng.choice([64, 80, 96, 128, 256]))
        group = quant == 8 and D % 32 == 0 and bool(rng.integers(0, 2))
        G = int(rng.choice([1, 2, 3, 4, 8, 16, 20]))
        B = int(rng.integers(1, 4))
        Hkv = int(rng.choice([1, 2, 4]))
        S = int(rng.integers(1, 80)) * r + int(rng.integers(0, r))
        cfg = dict(mode="jpeg", block_size=r, keep_freqs=k, quant_bits=quant)
        if group:
            cfg["quant_group"] = 32
        out.append((cfg, dt, B, Hkv, G, S, D))
    return out


JPEG_ATTN = _draw_jpeg(2028, 40)


@pytest.mark.parametrize("case", JPEG_ATTN, ids=[f"j{i}" for i in range(len(JPEG_ATTN))])
def test_jpeg_attention_sweep(case, oracle):
    cfg, dt, B, Hkv, G, S, D = case
    print(f"case jpeg sweep {case}", flush=True)
    ks, vs = build_streams(cfg, dt, B, Hkv, S, D, 500 + S, oracle)
    rng = np.random.default_rng(S + 3 * D)
    q = torch.from_numpy((rng.standard_normal((B, Hkv * G, 1, D)) / math.sqrt(D))
                         .astype(np.float32)).to(torch_dtype(dt)).to(DEV)
    out = fc.codec_decode_attention(q, ks, vs)
    assert_close(to_values(out)[:, :, 0], oracle_out(oracle, q, ks, vs, D ** -0.5), dt)


JPEG_STEPS = _draw_jpeg(2029, 16)


@pytest.mark.parametrize("case", JPEG_STEPS, ids=[f"t{i}" for i in range(len(JPEG_STEPS))])
def test_jpeg_step_sweep(case, oracle):
    """As test_png_step_sweep, on jpeg archives (int8 with one scale per row
    or per 32 features, or unquantised coefficients)."""
    _step_sweep(case, oracle)


def _draw_mixed(seed, n):
    """Cases whose queries have another dtype than the stream (png dense /
    packed, int8 jpeg, coefficient jpeg): the dispatch falls back to the
    pass that takes them."""
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        kind = i % 4
        r = int(rng.choice([4, 8, 16]))
        if kind == 0:
            cfg = dict(mode="png", block_size=r, keep_ratio=float(rng.choice([0.25, 1.0])))
        elif kind == 1:
            cfg = dict(mode="png", block_size=r, keep_ratio=0.5, packed=True)
        elif kind == 2:
            cfg = dict(mode="jpeg", block_size=r, keep_freqs=min(r, 4), quant_bits=8)
        else:
            cfg = dict(mode="jpeg", block_size=r, keep_freqs=min(r, 2))
        dts = ["f32", "f16", "bf16"]
        st_dt = str(rng.choice(dts))
        q_dt = str(rng.choice([d for d in dts if d != st_dt]))
        D = int(rng.choice([64, 128]))
        S = int(rng.integers(2, 60)) * r + int(rng.integers(0, r))
        out.append((cfg, st_dt, q_dt, int(rng.integers(1, 3)), int(rng.choice([1, 2])),
                    int(rng.choice([1, 2, 4, 8])), S, D))
    return out


MIXED = _draw_mixed(2031, 16)


@pytest.mark.parametrize("case", MIXED, ids=[f"m{i}" for i in range(len(MIXED))])
def test_mixed_dtype_attention_sweep(case, oracle):
    cfg, st_dt, q_dt, B, Hkv, G, S, D = case
    print(f"case mixed dtype sweep {case}", flush=True)
    ks, vs = build_streams(cfg, st_dt, B, Hkv, S, D, 300 + S, oracle)
    rng = np.random.default_rng(S + 7 * D)
    q = torch.from_numpy((rng.standard_normal((B, Hkv * G, 1, D)) / math.sqrt(D))
                         .astype(np.float32)).to(torch_dtype(q_dt)).to(DEV)
    out = fc.codec_decode_attention(q, ks, vs)
    assert out.dtype == q.dtype
    assert_close(to_values(out)[:, :, 0], oracle_out(oracle, q, ks, vs, D ** -0.5), q_dt)
