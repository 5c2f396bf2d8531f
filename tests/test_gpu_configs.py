"""GPU: the decode attention at the BASELINE configurations' own shapes, on
the kernel instantiations those configurations run, and through every entry
that reaches it (plain call, fused decode step, device-state step, graph
replay), each against the fp64 oracle on the streams' stored rows.

Tolerances are the contract's (fp16 / bf16: 2e-3 of max|ref| plus half an
ulp of the output dtype; fp32: 1e-5 absolute), as in test_gpu_attention.
"""

import math

import numpy as np
import pytest
import torch

import flashcodec_amd as fc
from flashcodec_amd import _native as N
from flashcodec_amd import attention as fa
from flashcodec_amd.cache import _CodecStream
from tests.conftest import to_values, torch_dtype
from tests.test_gpu_attention import assert_close, build_streams, oracle_out

pytestmark = pytest.mark.gpu
DEV = "cuda"
I8_C3 = dict(mode="jpeg", block_size=8, keep_freqs=4, quant_bits=8)


def queries(B, Hq, D, seed, dt):
    rng = np.random.default_rng(seed)
    q = (rng.standard_normal((B, Hq, 1, D)) / math.sqrt(D)).astype(np.float32)
    return torch.from_numpy(q).to(torch_dtype(dt)).to(DEV)


@pytest.fixture
def attention_pass():
    """use(name) selects the split pass for one test; restored afterwards."""
    prev = []

    def use(name):
        prev.append(N.set_attention_pass(name))
    yield use
    if prev:
        N.set_attention_pass(prev[0])


def test_c3_full_shape_every_sequence(oracle):
    """BASELINE C3 as bench.py runs it: B=8, 32 q / 8 kv heads, D=128,
    32768 archived tokens (r=8, k=4, int8) + 5 raw fp16 tokens, q fp16
    N(0,1)/sqrt(D); the default split count (64 head groups x 8 splits, one
    launch with the merge fused).  All 8 sequences against the oracle."""
    B, Hkv, G, D, S = 8, 8, 4, 128, 32768 + 5
    print("case c3 full shape", flush=True)
    ks, vs = build_streams(I8_C3, "f16", B, Hkv, S, D, 303, oracle)
    assert ks.n_blocks == 4096 and ks.raw.shape[-2] == 5
    q = queries(B, Hkv * G, D, 304, "f16")
    n_splits = N.lib().fc_attention_splits(N.STORE_JPEG_I8, N.F16, N.F16, 4, ks.n_blocks, B, Hkv,
                                           G, D, N.num_cus(q.device))
    assert 1 < n_splits <= 64                    # the fused (one-launch) merge
    out = fc.codec_decode_attention(q, ks, vs)
    ref = oracle_out(oracle, q, ks, vs, D ** -0.5)
    assert_close(to_values(out)[:, :, 0], ref, "f16")


def test_c5_attention_instantiation(oracle):
    """The decode attention of the C5 model's first decode step: bf16,
    16 q / 8 kv heads (G=2), D=128, k=4 int8, batch 16 over a 4096-token
    prompt plus the step's token (matrix-core pass <s=4, D=128, G=2>)."""
    B, Hkv, G, D, S = 16, 8, 2, 128, 4096 + 1
    print("case c5 attention shape", flush=True)
    ks, vs = build_streams(I8_C3, "bf16", B, Hkv, S, D, 505, oracle)
    q = queries(B, Hkv * G, D, 506, "bf16")
    out = fc.codec_decode_attention(q, ks, vs)
    assert_close(to_values(out)[:, :, 0], oracle_out(oracle, q, ks, vs, D ** -0.5), "bf16")


@pytest.mark.parametrize("dt,keep", [("f32", 0.25), ("f32", 1.0), ("bf16", 0.25)])
def test_c4_png_full_shape(dt, keep, oracle):
    """BASELINE C4: png fp32 (2, 8, 16384, 128), r=16, keep_ratio 0.25 and
    1.0, decode attention with 32 q heads (fp32 queries: 1e-5 absolute); and
    the same shape as a bf16 stream (bf16 anchors and queries, fp32 deltas)."""
    B, Hkv, G, D, S = 2, 8, 4, 128, 16384
    print(f"case c4 png keep={keep} {dt}", flush=True)
    cfg = dict(mode="png", block_size=16, keep_ratio=keep)
    ks, vs = build_streams(cfg, dt, B, Hkv, S, D, 404, oracle)
    assert ks.n_blocks == 1024 and ks.raw is None
    q = queries(B, Hkv * G, D, 405, dt)
    out = fc.codec_decode_attention(q, ks, vs)
    assert_close(to_values(out)[:, :, 0], oracle_out(oracle, q, ks, vs, D ** -0.5), dt)


@pytest.mark.parametrize("r,k,G,D", [(8, 2, 4, 128), (8, 4, 4, 128), (16, 16, 2, 64),
                                     (4, 1, 16, 128), (8, 8, 3, 64)])
def test_fp32_coefficient_archive_on_matrix_cores(r, k, G, D, oracle, attention_pass):
    """fp32 coefficient archives (quant_bits=0 in an fp32 model: the
    reference's default codec) on the png pass's fp32 products, many splits
    (B=2, 8 kv heads, 3000+ blocks and a raw tail): every sequence against
    the fp64 oracle (1e-5 absolute), and against the vector-ALU pass."""
    B, Hkv = 2, 8
    S = r * (24000 // r) + 5
    print(f"case fp32 coefficients r={r} k={k} G={G} D={D}", flush=True)
    cfg = dict(mode="jpeg", block_size=r, keep_freqs=k)
    ks, vs = build_streams(cfg, "f32", B, Hkv, S, D, 909 + k, oracle)
    q = queries(B, Hkv * G, D, 910 + k, "f32")
    n_splits = N.lib().fc_attention_splits(N.STORE_JPEG_FP, N.F32, N.F32, k, ks.n_blocks, B, Hkv,
                                           G, D, N.num_cus(q.device))
    assert n_splits > 1
    out = fc.codec_decode_attention(q, ks, vs)
    ref = oracle_out(oracle, q, ks, vs, D ** -0.5)
    assert_close(to_values(out)[:, :, 0], ref, "f32")
    attention_pass("valu")
    out_v = fc.codec_decode_attention(q, ks, vs)
    assert_close(to_values(out_v)[:, :, 0], ref, "f32")


@pytest.mark.parametrize("dt,G,D", [("f16", 4, 128), ("bf16", 2, 128), ("f16", 8, 64),
                                    ("bf16", 4, 256), ("f32", 4, 128), ("f32", 2, 256)])
def test_outlier_queries_on_matrix_cores(dt, G, D, oracle):
    """Queries with a few features 100x (and one head with a 1000x
    feature), the shape of real LLM queries: the matrix-core pass rounds each
    head's query to 14-bit integers relative to its largest element, which
    such heads stress most (fp32 queries: 30-bit integers, within the fp32
    contract's 1e-5)."""
    B, Hkv, S = 2, 2, 8 * 700 + 3
    print(f"case outlier queries {dt} G={G} D={D}", flush=True)
    ks, vs = build_streams(I8_C3, dt, B, Hkv, S, D, 606 + G + D, oracle)
    rng = np.random.default_rng(607)
    qn = (rng.standard_normal((B, Hkv * G, 1, D)) / math.sqrt(D)).astype(np.float32)
    for b in range(B):
        for h in range(Hkv * G):
            qn[b, h, 0, rng.choice(D, 4, replace=False)] *= 100.0
    qn[0, 0, 0, 3] = 1000.0 / math.sqrt(D)
    q = torch.from_numpy(qn).to(torch_dtype(dt)).to(DEV)
    out = fc.codec_decode_attention(q, ks, vs)
    assert_close(to_values(out)[:, :, 0], oracle_out(oracle, q, ks, vs, D ** -0.5), dt)


def test_impl_selectors_reference_style(oracle):
    """The reference's own check (tests/test_attention.py:100-115): impl
    "torch" and "triton" agree within 2e-3 on bf16 jpeg stores (int8 k=2,
    and unquantised k=4), "auto" returns the query dtype; here every
    selector runs the HIP kernels, so they also match the oracle."""
    torch.manual_seed(0)
    B, Hk, D, S, g = 1, 8, 128, 4096, 2
    k = torch.randn(B, Hk, S, D, device=DEV, dtype=torch.bfloat16)
    v = torch.randn(B, Hk, S, D, device=DEV, dtype=torch.bfloat16)
    q = torch.randn(B, Hk * g, 1, D, device=DEV, dtype=torch.bfloat16)
    for cfg in (dict(keep_freqs=2, quant_bits=8), dict(keep_freqs=4)):
        ks = _CodecStream(fc.make_codec("jpeg", block_size=8, **cfg))
        vs = _CodecStream(fc.make_codec("jpeg", block_size=8, **cfg))
        ks.append(k)
        vs.append(v)
        ref = fc.codec_decode_attention(q, ks, vs, impl="torch")
        tri = fc.codec_decode_attention(q, ks, vs, impl="triton")
        d = (ref.float() - tri.float()).abs().max().item()
        assert d < 2e-3, f"triton vs torch mismatch: {cfg} maxdiff={d:.2e}"
        auto = fc.codec_decode_attention(q, ks, vs)
        assert auto.dtype == q.dtype
        assert_close(to_values(auto)[:, :, 0], oracle_out(oracle, q, ks, vs, D ** -0.5), "bf16")


@pytest.mark.parametrize("cfg,dt,r", [(I8_C3, "f16", 8),
                                      (dict(mode="png", block_size=16, keep_ratio=1.0), "f32", 16)],
                         ids=["i8", "png"])
def test_static_pass_order_is_bitwise_reproducible(cfg, dt, r, oracle, attention_pass):
    """FC_PASS_STATIC: the matrix-core passes (int8 jpeg, png) with a fixed
    pass order give bitwise-equal outputs call after call, within tolerance
    of the oracle and of the queue-driven default."""
    B, Hkv, G, D, S = 2, 4, 4, 128, r * 2000 + 5
    ks, vs = build_streams(cfg, dt, B, Hkv, S, D, 808, oracle)
    q = queries(B, Hkv * G, D, 809, dt)
    auto = fc.codec_decode_attention(q, ks, vs)
    attention_pass("static")
    outs = [fc.codec_decode_attention(q, ks, vs) for _ in range(5)]
    for o in outs[1:]:
        assert torch.equal(o, outs[0])
    ref = oracle_out(oracle, q, ks, vs, D ** -0.5)
    assert_close(to_values(outs[0])[:, :, 0], ref, dt)
    assert_close(to_values(auto)[:, :, 0], ref, dt)


def test_merge_counters_return_to_zero(oracle):
    """The fused merge has no wait: every workgroup of a head group publishes
    its partial, waits until the stores are complete and then counts itself;
    the one that counts last merges and returns the group's counters to
    zero.  After int8 calls with 8, 5 and 8 splits and a png call, the
    counter region of every workspace (its first MiB) is zero again, and
    every output matches the oracle."""
    B, Hkv, G, D, S = 2, 4, 4, 128, 8 * 3000 + 5
    ks, vs = build_streams(I8_C3, "f16", B, Hkv, S, D, 909, oracle)
    q = queries(B, Hkv * G, D, 910, "f16")
    ref = oracle_out(oracle, q, ks, vs, D ** -0.5)
    for ns in (8, 5, 8):
        print(f"case merge counters int8 splits={ns}", flush=True)
        out = fc.codec_decode_attention(q, ks, vs, _n_splits=ns)
        assert_close(to_values(out)[:, :, 0], ref, "f16")
    print("case merge counters png", flush=True)
    P16 = dict(mode="png", block_size=16, keep_ratio=1.0)
    pk, pv = build_streams(P16, "f32", 1, 2, 16 * 400 + 3, D, 911, oracle)
    qp = queries(1, 2 * G, D, 912, "f32")
    out = fc.codec_decode_attention(qp, pk, pv)
    assert_close(to_values(out)[:, :, 0], oracle_out(oracle, qp, pk, pv, D ** -0.5), "f32")
    torch.cuda.synchronize()
    assert fa._WORKSPACES
    for ws in fa._WORKSPACES.values():
        words = ws[:1 << 20].view(torch.int32)
        assert int((words != 0).sum()) == 0


STEP_CFGS = [(I8_C3, "bf16", 2), (I8_C3, "f16", 4),
             (dict(mode="jpeg", block_size=8, keep_freqs=2), "f32", 4),
             (dict(mode="png", block_size=8, keep_ratio=0.5), "f16", 2),
             (dict(I8_C3, quant_group=32), "bf16", 2),
             (dict(I8_C3, keep_freqs=8), "f16", 4), (dict(I8_C3, keep_freqs=3), "bf16", 2),
             (dict(mode="png", block_size=16, keep_ratio=1.0), "f32", 4),
             (dict(mode="png", block_size=16, keep_ratio=0.25, packed=True), "f32", 4),
             (dict(mode="png", block_size=8, keep_ratio=0.5, packed=True), "bf16", 2),
             (dict(mode="jpeg", block_size=8, keep_freqs=4), "bf16", 2),
             (dict(mode="jpeg", block_size=8, keep_freqs=2), "f16", 4),
             (I8_C3, "f32", 2), (dict(I8_C3, quant_group=32), "f32", 4),
             (dict(mode="png", block_size=8, keep_ratio=0.5), "f32", 2),
             (dict(mode="png", block_size=4, keep_ratio=0.67), "f32", 8)]
STEP_IDS = ["i8-bf16", "i8-f16", "fp-f32", "png-f16", "i8g-bf16", "i8k8-f16", "i8k3-bf16",
            "png16-f32", "pngpk16-f32", "pngpk8-bf16", "fpj-bf16", "fpj-f16", "i8-f32",
            "i8g-f32", "png8-f32", "png4-f32"]


def _tokens(g, B, H, D, dt):
    """(B, H, 1, D) with the strides of an HF projection: (B, 1, H, D) transposed."""
    return torch.randn((B, 1, H, D), generator=g, device=DEV).to(torch_dtype(dt)).transpose(1, 2)


@pytest.mark.parametrize("cfg,dt,G", STEP_CFGS, ids=STEP_IDS)
def test_fused_decode_step_matches_oracle(cfg, dt, G, oracle):
    """codec_decode_step (token append + block archive + attention in one
    library call) against the oracle on the streams' rows after each step,
    across three block boundaries."""
    B, Hkv, D, r = 2, 2, 128, cfg["block_size"]
    print(f"case fused step vs oracle {cfg} {dt}", flush=True)
    ks, vs = build_streams(cfg, dt, B, Hkv, 5 * r + 3, D, 111, oracle)
    g = torch.Generator(device=DEV).manual_seed(112)
    for _ in range(3 * r + 1):
        q = _tokens(g, B, Hkv * G, D, dt)
        out = fc.codec_decode_step(q, _tokens(g, B, Hkv, D, dt), _tokens(g, B, Hkv, D, dt), ks, vs)
        assert_close(to_values(out)[:, :, 0], oracle_out(oracle, q, ks, vs, D ** -0.5), dt)


def _archives_equal(a, b):
    """Archive codes / scales / rows, tails and counters of two streams agree
    bit for bit."""
    assert a.n_blocks == b.n_blocks and a.seq_len == b.seq_len
    for x, y in zip(a._archive_tensors(), b._archive_tensors()):
        assert torch.equal(x[:, :, :a.n_blocks], y[:, :, :b.n_blocks])
    assert (a.raw is None) == (b.raw is None)
    if a.raw is not None:
        assert torch.equal(a.raw, b.raw)


C5 = dict(B=16, Hkv=8, G=2, D=128, dt="bf16")


C5_SCALES = [(I8_C3, N.STORE_JPEG_I8), (dict(I8_C3, quant_group=32), N.STORE_JPEG_I8G),
             (dict(mode="jpeg", block_size=8, keep_freqs=4), N.STORE_JPEG_FP)]
C5_SCALE_IDS = ["per-row", "per-32", "fp-coefficients"]


@pytest.mark.parametrize("cfg,kind", C5_SCALES, ids=C5_SCALE_IDS)
def test_fused_step_c5_scale_multi_split(cfg, kind, oracle):
    """The C5 model's per-layer decode step as it runs there: the one-launch
    step kernel (attn_split_i8_mfma<4, 128, 2, STEP>) at C5's geometry (batch
    16, 16 q / 8 kv heads, D=128, bf16, k=4: int8 with one scale per row or
    per 32 features, or the bf16 coefficients themselves) over 512 archived
    blocks + a 5-token tail, so the split count
    is the model's (4 > 1: the cross-split arrival and merge, the queued
    passes after the first and split 0's in-kernel append / archive beside
    streaming splits all run).  12 steps cross two block boundaries; after
    every step all 16 sequences are checked against the fp64 oracle on the
    streams' rows, and the archives the kernel wrote against the two-append
    path's, bit for bit."""
    B, Hkv, G, D, dt = C5["B"], C5["Hkv"], C5["G"], C5["D"], C5["dt"]
    r = 8
    S0 = 512 * r + 5
    print(f"case fused step at C5 scale {cfg}", flush=True)
    ks, vs = build_streams(cfg, dt, B, Hkv, S0, D, 141, oracle)
    ks_r, vs_r = build_streams(cfg, dt, B, Hkv, S0, D, 141, oracle)
    L = N.lib()
    g = torch.Generator(device=DEV).manual_seed(142)
    for step in range(r + 4):
        ns = L.fc_attention_splits(kind, N.BF16, N.BF16, 4, ks.n_blocks, B, Hkv, G, D,
                                   N.num_cus(torch.device(DEV)))
        assert 1 < ns <= 64, ns
        q = _tokens(g, B, Hkv * G, D, dt)
        k, v = _tokens(g, B, Hkv, D, dt), _tokens(g, B, Hkv, D, dt)
        out = fc.codec_decode_step(q, k, v, ks, vs)
        assert L.fc_last_step_single_launch() == 1
        ks_r.append(k)
        vs_r.append(v)
        _archives_equal(ks, ks_r)
        _archives_equal(vs, vs_r)
        assert_close(to_values(out)[:, :, 0], oracle_out(oracle, q, ks, vs, D ** -0.5), dt)


@pytest.mark.parametrize("D,k,dt", [(80, 4, "bf16"), (96, 8, "f16")])
def test_fused_decode_step_head_dims_80_96(D, k, dt, oracle):
    """The one-launch step on the matrix-core pass at head sizes that are not
    a multiple of 64 (products padded to 128 features) against the oracle."""
    B, Hkv, G, r = 2, 2, 4, 8
    cfg = dict(I8_C3, keep_freqs=k)
    print(f"case fused step D={D} k={k} {dt}", flush=True)
    ks, vs = build_streams(cfg, dt, B, Hkv, 6 * r + 2, D, 131 + D, oracle)
    g = torch.Generator(device=DEV).manual_seed(132)
    for _ in range(2 * r + 1):
        q = _tokens(g, B, Hkv * G, D, dt)
        out = fc.codec_decode_step(q, _tokens(g, B, Hkv, D, dt), _tokens(g, B, Hkv, D, dt), ks, vs)
        assert_close(to_values(out)[:, :, 0], oracle_out(oracle, q, ks, vs, D ** -0.5), dt)


class _Cache:
    """The part of an HF cache that graph.prepare reads: a list of codec layers."""

    def __init__(self, layers):
        self.layers = layers


def _codec_layer(cfg, ks, vs):
    from flashcodec_amd.cache import FlashCodecLayer
    layer = FlashCodecLayer(**cfg)
    layer._key_stream, layer._value_stream = ks, vs
    layer.codec = ks.codec
    return layer


@pytest.mark.parametrize("cfg,dt,G", STEP_CFGS, ids=STEP_IDS)
def test_graph_replayed_steps_match_oracle(cfg, dt, G, oracle):
    """One device-state decode step captured as a HIP graph and replayed
    with new query / key / value tokens copied into its input buffers: every
    replay's output against the oracle on the streams' rows (host counters
    advanced after each replay), with eager work between replays."""
    r = cfg["block_size"]
    print(f"case graph step vs oracle {cfg} {dt}", flush=True)
    _graph_steps(cfg, dt, 2, 2, G, 128, 4 * r + 5, 3 * r + 2, 222, oracle)


@pytest.mark.parametrize("cfg,kind", C5_SCALES, ids=C5_SCALE_IDS)
def test_graph_replayed_steps_c5_scale(cfg, kind, oracle):
    """Graph-replayed one-launch steps at C5's geometry (batch 16, 16 q / 8
    kv heads, D=128, bf16, k=4: int8 with one scale per row or per 32
    features, or bf16 coefficients; 512 archived blocks + 5 tail tokens: 4 splits, the model's):
    12 replays across two block boundaries, every sequence of every replay
    against the fp64 oracle, and the archives the replays wrote against the
    two-append path's, bit for bit."""
    print(f"case graph step at C5 scale {cfg}", flush=True)
    _graph_steps(cfg, C5["dt"], C5["B"], C5["Hkv"], C5["G"], C5["D"], 512 * 8 + 5, 12, 151,
                 oracle, check_archive=True, single_launch=True)


@pytest.mark.parametrize("dt,keep,packed", [("f32", 0.25, False), ("f32", 1.0, False),
                                            ("bf16", 0.25, False), ("f32", 0.25, True)])
def test_graph_replayed_steps_c4_scale(dt, keep, packed, oracle):
    """Graph-replayed one-launch png steps at C4's geometry (fp32 as C4, and
    bf16; batch 2, 32 q / 8 kv heads, D=128, r=16; 1024 archived blocks + 5
    tail tokens: the png pass's 32 splits): 14 replays across a block
    boundary, every sequence of every replay against the fp64 oracle, and
    the anchors and deltas the replays wrote against the two-append path's,
    bit for bit; and the packed Top-M archive at keep 0.25."""
    cfg = dict(mode="png", block_size=16, keep_ratio=keep, packed=packed)
    print(f"case graph step at C4 scale {cfg} {dt}", flush=True)
    _graph_steps(cfg, dt, 2, 8, 4, 128, 1024 * 16 + 5, 14, 161, oracle, check_archive=True,
                 single_launch=True)


def _graph_steps(cfg, dt, B, Hkv, G, D, S0, steps, seed, oracle, check_archive=False,
                 single_launch=False):
    pytest.importorskip("transformers")
    from flashcodec_amd import graph
    ks, vs = build_streams(cfg, dt, B, Hkv, S0, D, seed, oracle)
    if check_archive:
        ks_r, vs_r = build_streams(cfg, dt, B, Hkv, S0, D, seed, oracle)
    cache = _Cache([_codec_layer(cfg, ks, vs)])
    graph.prepare(cache, steps + 1)
    g = torch.Generator(device=DEV).manual_seed(seed + 1)
    q_in = torch.zeros((B, 1, Hkv * G, D), device=DEV, dtype=torch_dtype(dt)).transpose(1, 2)
    k_in = torch.zeros((B, 1, Hkv, D), device=DEV, dtype=torch_dtype(dt)).transpose(1, 2)
    v_in = torch.zeros_like(k_in)
    stream = torch.cuda.Stream()

    def fill():
        q_in.copy_(_tokens(g, B, Hkv * G, D, dt))
        k_in.copy_(_tokens(g, B, Hkv, D, dt))
        v_in.copy_(_tokens(g, B, Hkv, D, dt))

    def check():
        if check_archive:
            ks_r.append(k_in.clone())
            vs_r.append(v_in.clone())
            _archives_equal(ks, ks_r)
            _archives_equal(vs, vs_r)
        assert_close(to_values(out)[:, :, 0], oracle_out(oracle, q_in, ks, vs, D ** -0.5), dt)

    # one eager device-state step on the capture stream creates its workspace
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        fill()
        out = fc.codec_decode_step(q_in, k_in, v_in, ks, vs)
    torch.cuda.synchronize()
    if single_launch:
        assert N.lib().fc_last_step_single_launch() == 1
    graph.advance_host(cache)
    check()
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr, stream=stream):
        out = fc.codec_decode_step(q_in, k_in, v_in, ks, vs)
    for i in range(steps):
        fill()
        gr.replay()
        torch.cuda.synchronize()
        graph.advance_host(cache)
        check()
        _ = (torch.randn(64, 64, device=DEV) @ torch.randn(64, 64, device=DEV)).sum()
        torch.cuda.synchronize()
    graph.release(cache)                      # device counters == host counters, no overflow


@pytest.mark.parametrize("cfg,dt", [(I8_C3, "f16"),
                                    (dict(mode="png", block_size=8, keep_ratio=0.5), "f32"),
                                    (dict(mode="png", block_size=8, keep_ratio=1.0), "bf16"),
                                    (dict(mode="png", block_size=8, keep_ratio=0.5, packed=True),
                                     "bf16")],
                         ids=["i8", "png-f32", "png-bf16", "pngpk-bf16"])
def test_graph_step_past_reserved_capacity_is_reported(cfg, dt, oracle):
    """Device-state steps beyond the room prepare() reserved: the block that
    does not fit is not archived (the one-launch steps gate their in-kernel
    archive on the capacity), and release() reports it."""
    pytest.importorskip("transformers")
    from flashcodec_amd import graph
    B, Hkv, G, D, r = 1, 2, 2, 64, 8
    print(f"case step past capacity {cfg} {dt}", flush=True)
    ks, vs = build_streams(cfg, dt, B, Hkv, 16 * r, D, 333, oracle)
    assert ks.n_blocks == 16 and ks._capacity == 16
    cache = _Cache([_codec_layer(cfg, ks, vs)])
    graph.prepare(cache, 0)                   # room for one more block: 17 -> capacity 32
    g = torch.Generator(device=DEV).manual_seed(334)
    for _ in range(16 * r + 2 * r):           # 18 more blocks: two past the 32
        fc.codec_decode_step(_tokens(g, B, Hkv * G, D, dt), _tokens(g, B, Hkv, D, dt),
                             _tokens(g, B, Hkv, D, dt), ks, vs)
        assert N.lib().fc_last_step_single_launch() == 1
        graph.advance_host(cache)
    with pytest.raises(RuntimeError, match="capacity"):
        graph.release(cache)


def test_graph_decoder_refuses_steps_past_capacity():
    """GraphDecoder counts its steps and raises before a replay that would
    need archive room prepare() did not reserve."""
    pytest.importorskip("transformers")
    from flashcodec_amd import graph
    from tests.test_gpu_graph import prefill, tiny_qwen3
    model = tiny_qwen3(torch.float16, I8_C3)
    prompt = torch.randint(1, 512, (2, 19), generator=torch.Generator().manual_seed(3)).cuda()
    cache = prefill(model, prompt)
    dec = graph.GraphDecoder(model, cache, prompt[:, -1:], position=19, max_new_tokens=4,
                             warmup=1)
    toks = dec.generate(5)                    # 1 warm-up step + 4 replays
    assert toks.shape == (2, 5)
    with pytest.raises(RuntimeError, match="reserved"):
        dec.step()
    dec.close()


def test_c5_full_shape_materialization_free_tracks_materialized():
    """BASELINE C5's model at full shape (Qwen3-0.6B dims: 28 layers, hidden
    1024, 16 q / 8 kv heads, head_dim 128, bf16, random init), batch 16,
    4096-token prompt, 16 teacher-forced decode steps, jpeg r=8 k=4 int8:
    the materialisation-free logits track the materialised codec path (the
    reference's own semantics) and every layer takes the codec step."""
    pytest.importorskip("transformers")
    from transformers import Qwen3Config, Qwen3ForCausalLM
    cfg = Qwen3Config(vocab_size=151936, hidden_size=1024, intermediate_size=3072,
                      num_hidden_layers=28, num_attention_heads=16, num_key_value_heads=8,
                      head_dim=128, max_position_embeddings=8192, tie_word_embeddings=True)
    torch.manual_seed(0)
    with torch.device(DEV):
        model = Qwen3ForCausalLM(cfg).to(torch.bfloat16).eval()
    g = torch.Generator().manual_seed(1)
    B, P, steps = 16, 4096, 16
    ids = torch.randint(1, cfg.vocab_size, (B, P), generator=g).to(DEV)
    forced = torch.randint(1, cfg.vocab_size, (B, steps), generator=g).to(DEV)
    codec = dict(mode="jpeg", block_size=8, keep_freqs=4, quant_bits=8)

    def run(materialization_free):
        print(f"case c5 full shape, materialization_free={materialization_free}", flush=True)
        fc.apply_flash_codec(model, materialization_free=materialization_free, **codec)
        logits = []
        with torch.no_grad():
            out = model(input_ids=ids, use_cache=True, logits_to_keep=1)
            pkv = out.past_key_values
            for i in range(steps):
                pos = torch.full((B, 1), P + i, dtype=torch.long, device=DEV)
                out = model(input_ids=forced[:, i:i + 1], position_ids=pos, past_key_values=pkv,
                            use_cache=True, logits_to_keep=1)
                logits.append(out.logits[:, -1].float())
        counts = [getattr(m, "_flashcodec_codec_steps", 0)
                  for m in fc.find_attention_modules(model)]
        fc.remove_flash_codec(model)
        del pkv, out
        torch.cuda.empty_cache()
        return logits, counts

    ref, counts_m = run(False)
    got, counts_f = run(True)
    assert counts_m == [0] * 28
    assert counts_f == [steps] * 28, counts_f
    for i, (a, b) in enumerate(zip(ref, got)):
        err = (a - b).abs().max().item()
        assert err <= 3e-2 * a.abs().max().item(), (i, err)
