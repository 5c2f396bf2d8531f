#!/usr/bin/env python3
"""Benchmark of the north-star hot path on one MI355X.

Workload ("C3"): coefficient-domain split-K decode
attention, B=8, 32 query / 8 kv heads, D=128, 32768 archived tokens per
sequence (r=8, k=4, int8 K and V coefficients + fp32 scales) plus a raw tail
of 5 fp16 tokens; queries fp16 N(0,1)/sqrt(D); K/V synthetic AR(1) rho=0.95
fp16, archived by this package's own kernels before timing.

One step = one `codec_decode_attention` call on inputs resident in HBM: one
launch of the matrix-core split pass, whose last workgroup per head group
merges the split partials with the raw tail.  `value` is algorithmic GB/s of
the call:
  K+V int8 codes 2*134,217,728 + fp32 scales 2*4,194,304 + raw tails
  163,840 + q 65,536 + out 65,536 = 277,118,976 bytes per call.
The timed steps cycle over --sets copies of the archives (default 4, 1.1 GB:
more than the 256 MB last-level cache can hold, as a decode step cycles over
its layers' caches), so each call streams its archive from HBM; the same
launches repeated on one set (largely served by the last-level cache) are
reported as `single_set`.  The roofline object covers the kernel, each
launch timed with HIP events on the stream it is launched on.  Every
sequence of the output is checked against the fp64 CPU oracle (exit status
3 above the 2e-3 tolerance).  `cpu_baseline` times the reference's torch
CPU path (this build's restatement of flashcodec/attention.py:101-140,
oracle/torch_path.py) on all host cores for a bounded sample of the same
workload.

  python bench.py [--steps K] [--warmup W] [--gpus 1] [--sets N]
  python bench.py --mode copy     # plain copy, for PMC byte calibration
"""

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "coef-domain decode attn GB/s & % HBM peak; decode tokens/s at S=32K"
HBM_PEAK_GBS = 8000.0
B, HQ, HKV, D, S_ARCH, R, K, TAIL = 8, 32, 8, 128, 32768, 8, 4, 5
NB = S_ARCH // R
CODE_BYTES = B * HKV * NB * K * D              # per stream
SCALE_BYTES = B * HKV * NB * K * 4
Q_BYTES = B * HQ * D * 2
ALG_BYTES_CALL = 2 * CODE_BYTES + 2 * SCALE_BYTES + 2 * B * HKV * TAIL * D * 2 + 2 * Q_BYTES
PMC_SUMMARY = os.path.join(ROOT, "profiles", "attn_split_c3_pmc.md")


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def ar1_device(shape, rho, seed, device):
    """AR(1) along axis -2 with unit stationary variance, generated on the
    device with a chunked scan (256-token chunks, carries between chunks)."""
    import torch
    b, h, s, d = shape
    L = 256
    nch = (s + L - 1) // L
    g = torch.Generator(device=device).manual_seed(seed)
    eps = torch.randn((b, h, nch, L, d), generator=g, device=device)
    x = eps * math.sqrt(1.0 - rho * rho)
    x[:, :, 0, 0, :] = eps[:, :, 0, 0, :]
    for t in range(1, L):
        x[:, :, :, t, :] += rho * x[:, :, :, t - 1, :]
    pw = torch.tensor([rho ** (t + 1) for t in range(L)], device=device).view(L, 1)
    for c in range(1, nch):
        x[:, :, c] += pw * x[:, :, c - 1, L - 1:L, :]
    return x.reshape(b, h, nch * L, d)[:, :, :s]


def copy_mode(args):
    import torch
    n = args.copy_bytes
    src = torch.empty(n, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    src.fill_(1)
    for _ in range(args.warmup):
        dst.copy_(src)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(args.steps):
        dst.copy_(src)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / args.steps
    print(json.dumps({"mode": "copy", "bytes_per_copy": n, "ms_per_copy": ms,
                      "read_plus_write_GBs": 2 * n / ms / 1e6}))


def split_kernel_name(n_splits):
    """Kernel of this workload's call (int8 codes, 4 rows per block, D=128,
    groups of 4 q heads, no step, fp16 q, per-row scales): the matrix-core
    split pass, its merge fused in when the split count allows (one
    launch)."""
    from flashcodec_amd import _native as N
    from flashcodec_amd.attention import launches_per_call
    if N.lib().fc_get_attention_pass() == N.PASS_VECTOR:
        return "attn_split_kernel (merge fused)"
    if launches_per_call(N.STORE_JPEG_I8, n_splits) == 1:
        return "attn_split_i8_mfma<4,128,4,false,false,false> (merge fused)"
    return "attn_split_i8_mfma<4,128,4,false,false,false> + attn_merge_head_kernel"


def cpu_model():
    """Host CPU model name (/proc/cpuinfo), or None."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def torch_cpu_rate(fn, nbytes, reps=5, min_seconds=2.0):
    """(GB/s, cores) of fn() — the reference's torch CPU path restated in
    oracle/torch_path.py — on every affinity core of this host: the median
    of at least `reps` timed calls (more while under `min_seconds`) after
    one untimed call."""
    import statistics
    import torch
    cores = len(os.sched_getaffinity(0))
    prev = torch.get_num_threads()
    torch.set_num_threads(cores)
    fn()
    times = []
    t_start = time.perf_counter()
    while len(times) < reps or (time.perf_counter() - t_start < min_seconds and len(times) < 100):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    torch.set_num_threads(prev)
    return round(nbytes / statistics.median(times) / 1e9, 3), cores


SETTLE_S = 0.25  # untimed calls before the warm-up steps of each measurement


def settle(fn, seconds=SETTLE_S):
    """Calls fn(i), i = 0, 1, ..., untimed for at least `seconds` of device
    time.  The MI355X runs a new load below its steady rate for its first
    milliseconds: C3 calls measured 52.2 us each after 40 warm-up calls
    straight after setup and 49.9 us after 2000, the kernel alone 49.8 us
    in both runs.  Returns the number of calls."""
    import torch
    n = 0
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end:
        for _ in range(32):
            fn(n)
            n += 1
        torch.cuda.synchronize()
    return n


def timed(fn, steps, warmup):
    """Average ms of fn() over `steps` calls between events on the current
    stream, after `warmup` calls (and the untimed settle() period)."""
    import torch
    settle(lambda i: fn())
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def timed_cycle(fn, steps, warmup):
    """ms per call of fn(i), i = 0, 1, ..., between two events (after
    settle() and `warmup` calls)."""
    import torch
    settle(fn)
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(steps):
        fn(i)
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def c2_mode(args):
    """jpeg int8 archive + read of fp16 KV (B=4, H=32,
    S=8192, D=128), AR(1) rho=0.95 with a per-channel scale log-uniform in
    [0.1, 10]; r=8, k=4.  Bulk archive (fc_jpeg_encode of all 1024 blocks,
    one launch) and bulk read (fc_jpeg_decode of all blocks into an fp16
    view, one launch), algorithmic bytes per stream 268,435,456 (fp16 tokens)
    + 67,108,864 (codes) + 2,097,152 (fp32 scales); then the token-by-token
    append path of one stream."""
    import torch
    import flashcodec_amd as fc
    from flashcodec_amd import _native as N
    from flashcodec_amd.cache import _CodecStream
    from flashcodec_amd.codecs import jpeg as J
    dev = torch.device("cuda:0")
    b_, h_, s_, d_, r, k = 4, 32, 8192, 128, 8, 4
    nb = s_ // r
    g = torch.Generator(device=dev).manual_seed(2)
    scale = torch.exp(torch.empty((b_, h_, 1, d_), device=dev).uniform_(math.log(0.1), math.log(10.0),
                                                                       generator=g))
    x = (ar1_device((b_, h_, s_, d_), 0.95, 1, dev) * scale).to(torch.float16)
    coeffs = torch.empty((b_, h_, nb, k, d_), dtype=torch.int8, device=dev)
    scales = torch.empty((b_, h_, nb, k, 1), dtype=torch.float32, device=dev)
    out = torch.empty_like(x)
    alg = b_ * h_ * s_ * d_ * 2 + b_ * h_ * nb * k * d_ + b_ * h_ * nb * k * 4

    def archive():
        J.encode_into(x, r, k, 8, coeffs, scales, nb, 0, nb, s_)

    def read():
        J.decode_into(coeffs, scales, b_, h_, nb, 0, nb, d_, r, k, out, s_)

    t_arch = timed(archive, args.steps, args.warmup)
    t_read = timed(read, args.steps, args.warmup)
    log(f"bench c2: archive {t_arch * 1e3:.1f} us, read {t_read * 1e3:.1f} us")

    # token-by-token appends through the stream API (one token per call)
    n_tok = 512
    st = _CodecStream(fc.make_codec(mode="jpeg", block_size=r, keep_freqs=k, quant_bits=8))
    for t in range(16):                                  # warm the allocator and kernels
        st.append(x[:, :, t:t + 1])
    st = _CodecStream(fc.make_codec(mode="jpeg", block_size=r, keep_freqs=k, quant_bits=8))
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for t in range(n_tok):
        st.append(x[:, :, t:t + 1])
    torch.cuda.synchronize()
    t_tok = (time.perf_counter() - t0) / n_tok
    same = bool(torch.equal(st._coeffs[:, :, :n_tok // r], coeffs[:, :, :n_tok // r]) and
                torch.equal(st._scales[:, :, :n_tok // r], scales[:, :, :n_tok // r]))

    # the reference's torch CPU path (oracle/torch_path.py: dct_compress +
    # quantize, dequantize + dct_decompress + cast) on the whole workload,
    # every host core
    from oracle import torch_path as T
    basis = fc.dct_basis(r, k)
    xs = x.cpu()
    cq, sq = T.quantize(T.dct_compress(xs, r, basis))
    arch_gbs, cores = torch_cpu_rate(lambda: T.quantize(T.dct_compress(xs, r, basis)), alg)
    read_gbs, _ = torch_cpu_rate(
        lambda: T.dct_decompress(T.dequantize(cq, sq), r, basis).to(torch.float16), alg)
    cpu = {"unit": "GB/s", "cores": cores, "kind": "port", "cpu_model": cpu_model(),
           "sample": "the whole workload (128 sequences of 8192 tokens) through the "
                     "reference's torch CPU codec (restated in oracle/torch_path.py), median "
                     "of >= 5 calls",
           "archive": arch_gbs, "read": read_gbs}
    print(json.dumps({
        "metric": "jpeg int8 archive / read GB/s (C2)", "unit": "GB/s", "n_gpus": 1,
        "archive_GBs": round(alg / (t_arch * 1e-3) / 1e9, 1),
        "read_GBs": round(alg / (t_read * 1e-3) / 1e9, 1),
        "archive_us": round(t_arch * 1e3, 2), "read_us": round(t_read * 1e3, 2),
        "hbm_frac_archive": round(alg / (t_arch * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "hbm_frac_read": round(alg / (t_read * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "algorithmic_bytes": alg,
        "append_us_per_token": round(t_tok * 1e6, 2),
        "append_launches_per_token": "1 tail-row copy per token + 1 archive launch per 8 tokens",
        "token_by_token_codes_equal_bulk": same,
        "cpu_baseline": cpu,
        "config": {"workload": "C2 jpeg int8 archive + read", "B": b_, "H": h_, "S": s_, "D": d_,
                   "block": r, "keep_freqs": k, "dtype": "fp16"},
        "data": "synthetic AR(1) rho=0.95, per-channel scale log-uniform [0.1, 10]"}))


def step_timing(q, ks, vs, r, steps, warmup, g):
    """Decode steps on copies of the streams ks / vs: codec_decode_step
    (token append, the block archived every r-th step, attention; one launch
    where the store kind allows) against the reference's step (two appends,
    then the attention), each after 1024 untimed steps; room for every call
    reserved first, so no call regrows the archives.  us per step, and
    whether the step ran as one launch."""
    import torch
    import flashcodec_amd as fc
    from flashcodec_amd import _native as N
    B, H, D = ks._raw_buf.shape[0], ks._raw_buf.shape[1], q.shape[-1]
    kt = torch.randn((B, H, 1, D), generator=g, device=q.device).to(q.dtype)
    vt = torch.randn((B, H, 1, D), generator=g, device=q.device).to(q.dtype)
    n_pre = 1024
    out = {}
    for name in ("step", "append_attend"):
        sk, sv = archive_copy(ks), archive_copy(vs)
        for st_ in (sk, sv):
            st_._grow(st_.n_blocks + (n_pre + warmup + steps) // r + 2, kt)
        if name == "step":
            def fn():
                return fc.codec_decode_step(q, kt, vt, sk, sv)
        else:
            def fn():
                sk.append(kt)
                sv.append(vt)
                return fc.codec_decode_attention(q, sk, sv)
        for _ in range(n_pre + warmup):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        out[f"{name}_us"] = round(e0.elapsed_time(e1) / steps * 1e3, 2)
        if name == "step":
            out["step_single_launch"] = N.lib().fc_last_step_single_launch() == 1
        del sk, sv, fn
    return out


def c4_mode(args):
    """png mode on fp32 KV (B=2, H=8, S=16384, D=128),
    AR(1) rho=0.98, r=16, keep_ratio 0.25 (4 of 15 deltas) and 1.0.  Bulk
    archive and bulk read of one stream (algorithmic bytes 134,217,728 fp32
    tokens + 125,829,120 fp32 deltas + 8,388,608 fp32 anchors), and decode
    attention of 32 query heads (one fp32 query token per sequence) over K
    and V archives (268,435,456 bytes of stored rows + q + out); keep_ratio
    1.0 is checked against dense fp32 attention over the original tokens."""
    import torch
    import flashcodec_amd as fc
    from flashcodec_amd.cache import _CodecStream
    from flashcodec_amd.codecs import png as P
    dev = torch.device("cuda:0")
    b_, h_, s_, d_, r, hq = 2, 8, 16384, 128, 16, 32
    nb = s_ // r
    x = {"k": ar1_device((b_, h_, s_, d_), 0.98, 1, dev), "v": ar1_device((b_, h_, s_, d_), 0.98, 2, dev)}
    g = torch.Generator(device=dev).manual_seed(3)
    q = torch.randn((b_, hq, 1, d_), generator=g, device=dev) / math.sqrt(d_)
    alg_codec = b_ * h_ * s_ * d_ * 4 + b_ * h_ * nb * (r - 1) * d_ * 4 + b_ * h_ * nb * d_ * 4
    alg_attn = 2 * b_ * h_ * nb * r * d_ * 4 + 2 * b_ * hq * d_ * 4
    res = {"metric": "png archive / read / decode attention (C4)", "unit": "GB/s", "n_gpus": 1,
           "config": {"workload": "C4 png", "B": b_, "H": h_, "S": s_, "D": d_, "block": r,
                      "q_heads": hq, "dtype": "fp32"},
           "data": "synthetic AR(1) rho=0.98", "algorithmic_bytes_codec": alg_codec,
           "algorithmic_bytes_attention": alg_attn}
    for keep in (0.25, 1.0):
        codec = fc.make_codec(mode="png", block_size=r, keep_ratio=keep)
        m_keep = codec.keep_m
        deltas = torch.empty((b_, h_, nb, r - 1, d_), dtype=torch.float32, device=dev)
        anchors = torch.empty((b_, h_, nb, d_), dtype=torch.float32, device=dev)
        out = torch.empty_like(x["k"])

        def archive():
            P.encode_into(x["k"], r, m_keep, deltas, anchors, nb, 0, nb, s_)

        def read():
            P.decode_into(deltas, anchors, b_, h_, nb, 0, nb, d_, r, out, s_)

        t_arch = timed(archive, args.steps, args.warmup)
        t_read = timed(read, args.steps, args.warmup)
        ks, vs = _CodecStream(codec), _CodecStream(codec)
        ks.append(x["k"])
        vs.append(x["v"])
        t_attn = timed(lambda: fc.codec_decode_attention(q, ks, vs), args.steps, args.warmup)
        # the same calls cycling over 4 copies of the archives (1.07 GB, beyond
        # the 256 MB last-level cache), as a decode step cycles over layers
        sets = [(ks, vs)] + [(archive_copy(ks), archive_copy(vs)) for _ in range(3)]
        t_rot = timed_cycle(lambda i: fc.codec_decode_attention(q, *sets[i % 4]), args.steps,
                            args.warmup)
        del sets
        torch.cuda.empty_cache()
        tag = f"keep{keep}"
        res[tag] = {"archive_GBs": round(alg_codec / (t_arch * 1e-3) / 1e9, 1),
                    "read_GBs": round(alg_codec / (t_read * 1e-3) / 1e9, 1),
                    "attention_GBs": round(alg_attn / (t_attn * 1e-3) / 1e9, 1),
                    "attention_rotating_GBs": round(alg_attn / (t_rot * 1e-3) / 1e9, 1),
                    "archive_us": round(t_arch * 1e3, 2), "read_us": round(t_read * 1e3, 2),
                    "attention_us": round(t_attn * 1e3, 2),
                    "attention_rotating_us": round(t_rot * 1e3, 2), "kept_deltas": m_keep}
        if keep == 1.0:
            o = fc.codec_decode_attention(q, ks, vs)
            G = hq // h_
            kk = x["k"].repeat_interleave(G, dim=1)
            vv = x["v"].repeat_interleave(G, dim=1)
            p_ = torch.softmax((q @ kk.transpose(-1, -2).contiguous()) * d_ ** -0.5, dim=-1)
            ref = p_ @ vv
            res[tag]["vs_dense_max_abs_err"] = float((o - ref).abs().max())
        # the reference's torch CPU path (oracle/torch_path.py) on every host
        # core: png_filter / png_reconstruct of the whole stream; decode
        # attention (png rows, fp32) on one of the 16 (batch, kv head)
        # sequences with its 4 query heads
        from oracle import torch_path as T
        xs = x["k"].cpu()
        dl, an = T.png_filter(xs, r, keep)
        arch_gbs, cores = torch_cpu_rate(lambda: T.png_filter(xs, r, keep), alg_codec)
        read_gbs, _ = torch_cpu_rate(lambda: T.png_reconstruct(dl, an), alg_codec)
        rk = T.png_rows(ks._deltas[:1, :1, :nb].cpu(), ks._anchors[:1, :1, :nb].cpu())
        rv = T.png_rows(vs._deltas[:1, :1, :nb].cpu(), vs._anchors[:1, :1, :nb].cpu())
        qs = q[:1, :hq // h_].cpu()
        A = torch.tril(torch.ones(r, r))
        attn_gbs, _ = torch_cpu_rate(
            lambda: T.decode_attention(qs, rk, rv, None, None, A, d_ ** -0.5),
            alg_attn // (b_ * h_))
        res[tag]["cpu_baseline"] = {
            "unit": "GB/s", "cores": cores, "kind": "port", "cpu_model": cpu_model(),
            "sample": "archive / read: the whole stream; attention: 1 of the 16 (batch, kv "
                      "head) sequences (16384 tokens, 4 query heads); the reference's torch CPU "
                      "path (restated in oracle/torch_path.py), median of >= 5 calls",
            "archive": arch_gbs, "read": read_gbs, "attention": attn_gbs}
        res[tag].update(step_timing(q, ks, vs, r, args.steps, args.warmup, g))
        torch.cuda.empty_cache()
        log(f"bench c4 keep {keep}: {res[tag]}")

    # packed Top-M archives (this build's fixed-rate format; the reference
    # stores the same deltas dense): archive, read and decode attention
    for keep in (0.25, 0.5):
        codec = fc.make_codec(mode="png", block_size=r, keep_ratio=keep, packed=True)
        m_keep = codec.keep_m
        vals = torch.empty((b_, h_, nb, m_keep, d_), dtype=torch.float32, device=dev)
        masks = torch.empty((b_, h_, nb, d_), dtype=torch.int32, device=dev)
        anchors = torch.empty((b_, h_, nb, d_), dtype=torch.float32, device=dev)
        out = torch.empty_like(x["k"])
        store = b_ * h_ * nb * d_ * 4 * (m_keep + 2)          # values + mask words + anchors
        alg_pk_codec = b_ * h_ * s_ * d_ * 4 + store
        alg_pk_attn = 2 * store + 2 * b_ * hq * d_ * 4

        def archive_pk():
            P.encode_packed_into(x["k"], r, m_keep, vals, masks, anchors, nb, 0, nb, s_)

        def read_pk():
            P.decode_packed_into(vals, masks, anchors, b_, h_, nb, 0, nb, d_, r, m_keep, out, s_)

        t_arch = timed(archive_pk, args.steps, args.warmup)
        t_read = timed(read_pk, args.steps, args.warmup)
        ks, vs = _CodecStream(codec), _CodecStream(codec)
        ks.append(x["k"])
        vs.append(x["v"])
        t_attn = timed(lambda: fc.codec_decode_attention(q, ks, vs), args.steps, args.warmup)
        sets = [(ks, vs)] + [(archive_copy(ks), archive_copy(vs)) for _ in range(7)]
        t_rot = timed_cycle(lambda i: fc.codec_decode_attention(q, *sets[i % 8]), args.steps,
                            args.warmup)
        del sets
        torch.cuda.empty_cache()
        steps_pk = step_timing(q, ks, vs, r, args.steps, args.warmup, g)
        res[f"packed_keep{keep}"] = {
            "kept_deltas": m_keep, "store_bytes_per_stream": store,
            "dense_store_bytes_per_stream": b_ * h_ * nb * d_ * 4 * r,
            "archive_GBs": round(alg_pk_codec / (t_arch * 1e-3) / 1e9, 1),
            "read_GBs": round(alg_pk_codec / (t_read * 1e-3) / 1e9, 1),
            "attention_GBs": round(alg_pk_attn / (t_attn * 1e-3) / 1e9, 1),
            "attention_rotating_GBs": round(alg_pk_attn / (t_rot * 1e-3) / 1e9, 1),
            "attention_rotating_hbm_frac": round(alg_pk_attn / (t_rot * 1e-3) / 1e9 / HBM_PEAK_GBS,
                                                 4),
            "archive_us": round(t_arch * 1e3, 2), "read_us": round(t_read * 1e3, 2),
            "attention_us": round(t_attn * 1e3, 2), "attention_rotating_us": round(t_rot * 1e3, 2),
            "algorithmic_bytes_attention": alg_pk_attn,
            "cpu_baseline": "the reference stores these deltas dense: see keep0.25 (same rows)",
            **steps_pk}
        log(f"bench c4 packed keep {keep}: {res[f'packed_keep{keep}']}")

    # the same shape as a bf16 / fp16 stream (16-bit anchors and queries, fp32
    # deltas), keep 0.25: the png matrix-core pass against the vector-ALU pass,
    # over 4 rotating archive sets
    from flashcodec_amd import _native as N
    for dname, dt in (("bf16", torch.bfloat16), ("f16", torch.float16)):
        codec = fc.make_codec(mode="png", block_size=r, keep_ratio=0.25)
        ks, vs = _CodecStream(codec), _CodecStream(codec)
        ks.append(x["k"].to(dt))
        vs.append(x["v"].to(dt))
        q16 = q.to(dt)
        alg16 = 2 * b_ * h_ * nb * (d_ * 2 + (r - 1) * d_ * 4) + 2 * b_ * hq * d_ * 2
        sets = [(ks, vs)] + [(archive_copy(ks), archive_copy(vs)) for _ in range(3)]
        t16 = {}
        for pname in ("auto", "valu"):
            prev = N.set_attention_pass(pname)
            t16[pname] = timed_cycle(lambda i: fc.codec_decode_attention(q16, *sets[i % 4]),
                                     args.steps, args.warmup)
            N.set_attention_pass(prev)
        del sets, ks, vs
        torch.cuda.empty_cache()
        res[f"{dname}_keep0.25"] = {
            "algorithmic_bytes_attention": alg16,
            "attention_rotating_us": round(t16["auto"] * 1e3, 2),
            "attention_rotating_GBs": round(alg16 / (t16["auto"] * 1e-3) / 1e9, 1),
            "attention_rotating_hbm_frac": round(alg16 / (t16["auto"] * 1e-3) / 1e9 / HBM_PEAK_GBS,
                                                 4),
            "vector_alu_pass_rotating_us": round(t16["valu"] * 1e3, 2)}
        log(f"bench c4 {dname}: {res[f'{dname}_keep0.25']}")
    print(json.dumps(res))


def c1_mode(args):
    """jpeg round trip of fp32 KV (B=1, H=8, S=4096,
    D=128), each (b, h, d) channel AR(1) rho=0.97 with unit variance; r=8,
    k=2, no quantization; encode all 512 blocks, then read(); PSNR
    (20 log10(max|x| / rmse)) and max abs error, and the reconstruction
    compared bit for bit with the CPU oracle."""
    import numpy as np
    import torch
    import flashcodec_amd as fc
    from flashcodec_amd.cache import _CodecStream
    from oracle import oracle as O
    dev = torch.device("cuda:0")
    b_, h_, s_, d_, r, k = 1, 8, 4096, 128, 8, 2
    x = ar1_device((b_, h_, s_, d_), 0.97, 1, dev)
    st = _CodecStream(fc.make_codec(mode="jpeg", block_size=r, keep_freqs=k))
    st.append(x)
    rec = st.read()
    err = (rec - x).float()
    rmse = float(err.pow(2).mean().sqrt())
    psnr = 20 * math.log10(float(x.abs().max()) / rmse)
    basis = fc.dct_basis(r, k).numpy()
    xn = x.cpu().numpy()
    coef = O.jpeg_encode(xn, r, k, basis, "f32")
    ref = O.jpeg_decode(coef, r, basis, "f32")
    # the reference's torch CPU path (oracle/torch_path.py), every host core
    from oracle import torch_path as T
    bt = fc.dct_basis(r, k)
    xc = x.cpu()
    ct = T.dct_compress(xc, r, bt)
    alg_c = b_ * h_ * s_ * d_ * 4 + b_ * h_ * (s_ // r) * k * d_ * 4
    arch_gbs, cores = torch_cpu_rate(lambda: T.dct_compress(xc, r, bt), alg_c)
    read_gbs, _ = torch_cpu_rate(lambda: T.dct_decompress(ct, r, bt), alg_c)
    cpu = {"unit": "GB/s", "cores": cores, "kind": "port", "cpu_model": cpu_model(),
           "sample": "the whole C1 stream through the reference's torch CPU codec (restated in "
                     "oracle/torch_path.py), median of >= 5 calls",
           "archive": arch_gbs, "read": read_gbs}
    bit_exact = bool(np.array_equal(rec.cpu().numpy().view(np.uint32), np.asarray(ref, np.float32).view(np.uint32)))
    alg = b_ * h_ * s_ * d_ * 4 + b_ * h_ * (s_ // r) * k * d_ * 4
    t_arch = timed(lambda: _CodecStream(st.codec).append(x), args.steps, args.warmup)
    print(json.dumps({"metric": "jpeg fp32 round trip accuracy (C1)", "psnr_db": round(psnr, 3),
                      "max_abs_err": float(err.abs().max()), "rmse": rmse,
                      "bit_exact_vs_oracle": bit_exact,
                      "archive_us": round(t_arch * 1e3, 2),
                      "archive_GBs": round(alg / (t_arch * 1e-3) / 1e9, 1),
                      "cpu_baseline": cpu,
                      "config": {"workload": "C1 jpeg round trip", "B": b_, "H": h_, "S": s_, "D": d_,
                                 "block": r, "keep_freqs": k, "dtype": "fp32"},
                      "data": "synthetic AR(1) rho=0.97, unit variance"}))


def refshapes_mode(args):
    """The reference's published decode-attention timings (flashcodec
    README.md:318-325: Triton split-K 0.09 ms at S=16384 and 0.16 ms at
    S=65536; one layer, B=1, Hkv=8, Hq=16, D=128, jpeg r=8 k=2 int8, on an
    unstated CUDA GPU) against this build on the same shapes."""
    import torch
    import flashcodec_amd as fc
    from flashcodec_amd.cache import _CodecStream
    dev = torch.device("cuda:0")
    res = {"metric": "decode attention ms at the reference's published shapes", "unit": "ms",
           "reference_ms": {"16384": 0.09, "65536": 0.16}, "ours": {}}
    for s_ in (16384, 65536):
        cfg = dict(mode="jpeg", block_size=8, keep_freqs=2, quant_bits=8)
        ks, vs = _CodecStream(fc.make_codec(**cfg)), _CodecStream(fc.make_codec(**cfg))
        for st, seed in ((ks, 1), (vs, 2)):
            st.append(ar1_device((1, 8, s_, 128), 0.95, seed, dev).to(torch.float16))
        q = (torch.randn((1, 16, 1, 128), device=dev) / math.sqrt(128)).to(torch.float16)
        ms = timed(lambda: fc.codec_decode_attention(q, ks, vs), args.steps, args.warmup)
        nbytes = 2 * (1 * 8 * (s_ // 8) * 2 * 128 + 1 * 8 * (s_ // 8) * 2 * 4)
        res["ours"][str(s_)] = {"ms": round(ms, 4), "GBs": round(nbytes / (ms * 1e-3) / 1e9, 1),
                                "speedup_vs_reference": round(res["reference_ms"][str(s_)] / ms, 2)}
    print(json.dumps(res))


def shapes_mode(args):
    """Decode attention at C3's geometry (B=8, 32 q / 8 kv heads, 32768
    archived + 5 raw tokens, r=8) on int8 archives (fp16 stream) for head
    sizes, keep_freqs, per-32 scales and fp32 queries besides C3's, and on
    fp16 / bf16 / fp32 coefficient archives (quant_bits=0): each on the
    matrix-core pass (FC_PASS_AUTO) and on the vector-ALU pass
    (FC_PASS_VECTOR), one archive set, max error vs the fp64 oracle over all
    sequences."""
    import torch
    import flashcodec_amd as fc
    from flashcodec_amd import _native as N
    from flashcodec_amd.cache import _CodecStream
    dev = torch.device("cuda:0")
    res = {"metric": "decode attention GB/s by head size, keep_freqs and store, jpeg, C3 geometry",
           "unit": "GB/s", "shapes": []}
    prev = N.lib().fc_get_attention_pass()
    # (D, keep_freqs, quantizer group, query dtype, quant_bits): int8 rows
    # (fp16 stream) and fp coefficient rows in the query's dtype
    for D, k, grp, qdt, qb in ((128, 3, 0, "f16", 8), (128, 8, 0, "f16", 8), (80, 4, 0, "f16", 8),
                               (96, 4, 0, "f16", 8), (128, 4, 32, "f16", 8), (96, 4, 32, "f16", 8),
                               (128, 4, 0, "f32", 8), (128, 4, 32, "f32", 8),
                               (128, 4, 0, "f16", 0), (128, 2, 0, "bf16", 0),
                               (128, 4, 0, "f32", 0), (128, 2, 0, "f32", 0),
                               (128, 4, 0, "f16", 8)):
        cfg = dict(mode="jpeg", block_size=R, keep_freqs=k, quant_bits=qb)
        if grp:
            cfg["quant_group"] = grp
        qt = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}[qdt]
        st_dt = torch.float16 if qb else qt
        ks, vs = _CodecStream(fc.make_codec(**cfg)), _CodecStream(fc.make_codec(**cfg))
        for st, seed in ((ks, 1), (vs, 2)):
            x = ar1_device((B, HKV, S_ARCH + TAIL, D), 0.95, seed, dev).to(st_dt)
            st.append(x)
            del x
        g = torch.Generator(device=dev).manual_seed(3)
        q = (torch.randn((B, HQ, 1, D), generator=g, device=dev) / math.sqrt(D)).to(qt)
        st_es = torch.empty((), dtype=st_dt).element_size()
        row_bytes = D + 4 * (D // grp if grp else 1) if qb else st_es * D
        qo_bytes = 2 * B * HQ * D * q.element_size()
        nbytes = 2 * (B * HKV * NB * k * row_bytes) + 2 * B * HKV * TAIL * D * st_es + qo_bytes
        row = {"D": D, "keep_freqs": k, "quant_bits": qb, "quant_group": grp, "q_dtype": qdt,
               "algorithmic_bytes": nbytes}
        for name, code in (("matrix_core", N.PASS_AUTO), ("vector_alu", N.PASS_VECTOR)):
            N.lib().fc_set_attention_pass(code)
            ms = timed(lambda: fc.codec_decode_attention(q, ks, vs), args.steps, args.warmup)
            out = fc.codec_decode_attention(q, ks, vs)
            err, _ = check_against_oracle(q, ks, vs, out)
            row[name] = {"us": round(ms * 1e3, 2), "GBs": round(nbytes / (ms * 1e-3) / 1e9, 1),
                         "max_rel_err": err}
        N.lib().fc_set_attention_pass(prev)
        res["shapes"].append(row)
        log(f"bench shapes: {row}")
        del ks, vs
        torch.cuda.empty_cache()
    print(json.dumps(res))


def c5_mode(args):
    """end-to-end greedy decoding through the attention
    patch on a randomly initialised Qwen3-0.6B-shaped decoder (28 layers,
    hidden 1024, 16 q / 8 kv heads, head_dim 128, intermediate 3072, vocab
    151936, tied embeddings, bf16): batch 16, 4096 random prompt ids, 256
    decode steps, jpeg r=8 k=4 int8 with materialization-free attention,
    against the same model with transformers' own KV cache.  Also batch 1,
    4096 + 32 (the setting of flashcodec README.md:334-343: 40.3 tok/s
    materialization-free on an unstated CUDA GPU)."""
    import torch
    import flashcodec_amd as fc
    from transformers import Qwen3Config, Qwen3ForCausalLM
    dev = torch.device("cuda:0")
    cfg = Qwen3Config(vocab_size=151936, hidden_size=1024, intermediate_size=3072,
                      num_hidden_layers=28, num_attention_heads=16, num_key_value_heads=8,
                      head_dim=128, max_position_embeddings=8192, tie_word_embeddings=True)
    torch.manual_seed(0)
    model = Qwen3ForCausalLM(cfg).to(device=dev, dtype=torch.bfloat16).eval()
    model.generation_config.eos_token_id = None
    # --c5-group 32: archives with one scale per 32 features
    qgroup = {"quant_group": args.c5_group} if args.c5_group else {}

    def run(batch, prompt, steps):
        g = torch.Generator().manual_seed(1)
        ids = torch.randint(1, cfg.vocab_size, (batch, prompt), generator=g).to(dev)
        with torch.no_grad():
            # memory as flashcodec benchmarks/bench_e2e.py:68-80 reports it:
            # peak = most allocated during the run, steady = still allocated
            # after it (the cache), both above what was allocated before
            torch.cuda.synchronize()
            torch.cuda.empty_cache()
            torch.cuda.reset_peak_memory_stats()
            base = torch.cuda.memory_allocated()
            t0 = time.perf_counter()
            out = model(input_ids=ids, use_cache=True, logits_to_keep=1)
            pkv = out.past_key_values
            nxt = out.logits[:, -1].argmax(-1, keepdim=True)
            torch.cuda.synchronize()
            t1 = time.perf_counter()
            for _ in range(steps):
                out = model(input_ids=nxt, past_key_values=pkv, use_cache=True, logits_to_keep=1)
                pkv = out.past_key_values
                nxt = out.logits[:, -1].argmax(-1, keepdim=True)
            torch.cuda.synchronize()
            t2 = time.perf_counter()
            del out
            mem = {"peak_MB": round((torch.cuda.max_memory_allocated() - base) / 1e6, 1),
                   "steady_MB": round((torch.cuda.memory_allocated() - base) / 1e6, 1)}
            del pkv, nxt
        if steps == 0:
            return {"prefill_s": round(t1 - t0, 4), **mem}
        return {"prefill_s": round(t1 - t0, 4), "decode_ms_per_step": round((t2 - t1) / steps * 1e3, 3),
                "decode_tokens_per_s": round(batch * steps / (t2 - t1), 1), **mem}

    def run_graph(batch, prompt, steps, warmup=2):
        """Prefill eagerly, then `steps` greedy decode steps of which the
        first `warmup` run eagerly and the rest replay a captured HIP graph
        of one step (flashcodec_amd.graph); decode time over the replays."""
        from flashcodec_amd import graph
        g = torch.Generator().manual_seed(1)
        ids = torch.randint(1, cfg.vocab_size, (batch, prompt), generator=g).to(dev)
        with torch.no_grad():
            out = model(input_ids=ids, use_cache=True, logits_to_keep=1)
            nxt = out.logits[:, -1].argmax(-1, keepdim=True)
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            dec = graph.GraphDecoder(model, out.past_key_values, nxt, position=prompt,
                                     max_new_tokens=steps, warmup=warmup)
            torch.cuda.synchronize()
            t1 = time.perf_counter()
            dec.generate(warmup)
            for _ in range(steps - warmup):
                dec.step()
            torch.cuda.synchronize()
            t2 = time.perf_counter()
            dec.close()
        n = steps - warmup
        return {"warmup_and_capture_s": round(t1 - t0, 4),
                "decode_ms_per_step": round((t2 - t1) / n * 1e3, 3),
                "decode_tokens_per_s": round(batch * n / (t2 - t1), 1), "graph_steps": n}

    def run_graph_raw(batch, prompt, steps, warmup=2):
        """The same decode on raw KV in transformers' StaticCache (preallocated
        for the whole run, written in place) with each step replayed from a
        captured HIP graph: the baseline on equal footing with run_graph."""
        from transformers import StaticCache
        g = torch.Generator().manual_seed(1)
        ids = torch.randint(1, cfg.vocab_size, (batch, prompt), generator=g).to(dev)
        cache = StaticCache(config=model.config, max_cache_len=prompt + steps + 1)
        with torch.no_grad():
            out = model(input_ids=ids, past_key_values=cache, use_cache=True, logits_to_keep=1,
                        cache_position=torch.arange(prompt, device=dev))
            tok = out.logits[:, -1].argmax(-1, keepdim=True)
            pos = torch.full((batch, 1), prompt, dtype=torch.long, device=dev)
            cpos = torch.tensor([prompt], dtype=torch.long, device=dev)
            stream = torch.cuda.Stream(device=dev)

            def fwd():
                return model(input_ids=tok, position_ids=pos, cache_position=cpos,
                             past_key_values=cache, use_cache=True, logits_to_keep=1).logits

            def advance(logits):
                tok.copy_(logits[:, -1].argmax(-1, keepdim=True))
                pos.add_(1)
                cpos.add_(1)

            torch.cuda.synchronize()
            t0 = time.perf_counter()
            stream.wait_stream(torch.cuda.current_stream(dev))
            with torch.cuda.stream(stream):
                for _ in range(warmup):
                    advance(fwd())
            torch.cuda.current_stream(dev).wait_stream(stream)
            torch.cuda.synchronize()
            gr = torch.cuda.CUDAGraph()
            with torch.cuda.graph(gr, stream=stream):
                logits = fwd()
            torch.cuda.synchronize()
            t1 = time.perf_counter()
            with torch.cuda.stream(stream):
                for _ in range(steps - warmup):
                    gr.replay()
                    advance(logits)
            torch.cuda.synchronize()
            t2 = time.perf_counter()
        n = steps - warmup
        del gr, cache
        torch.cuda.empty_cache()
        return {"warmup_and_capture_s": round(t1 - t0, 4),
                "decode_ms_per_step": round((t2 - t1) / n * 1e3, 3),
                "decode_tokens_per_s": round(batch * n / (t2 - t1), 1), "graph_steps": n}

    if args.c5_graph:
        # raw KV (StaticCache) and codec decoding, each step replayed from a
        # captured HIP graph
        raw = {}
        for tag, (bt, pr, st) in (("raw_static_graph_b16", (16, 4096, 256)),
                                  ("raw_static_graph_b1", (1, 4096, 32))):
            try:
                raw[tag] = run_graph_raw(bt, pr, st)
            except Exception as exc:         # a baseline that cannot be captured is reported
                raw[tag] = {"error": f"{type(exc).__name__}: {exc}"[:300]}
            log(f"bench c5 graph: {tag} {raw[tag]}")
        fc.apply_flash_codec(model, mode="jpeg", block_size=8, keep_freqs=4, quant_bits=8, **qgroup,
                             materialization_free=True)
        run(2, 64, 4)
        res = {"metric": "end-to-end decode tokens/s (C5), codec, HIP-graph decode steps",
               "unit": "tokens/s", "n_gpus": 1,
               "codec_graph_b16": run_graph(16, 4096, 256),
               "codec_graph_b1": run_graph(1, 4096, 32), **raw}
        res["value"] = res["codec_graph_b16"]["decode_tokens_per_s"]
        log(f"bench c5 graph: {res}")
        print(json.dumps(res))
        return

    if args.c5_steps is not None:
        # one run of the named setting (for kernel traces: launches per step
        # are the dispatch count of a run minus that of the same run with 0
        # steps, divided by the steps)
        if args.c5_kv != "raw":
            fc.apply_flash_codec(model, mode="jpeg", block_size=8, keep_freqs=4, quant_bits=8, **qgroup,
                                 materialization_free=True)
        if args.c5_kv == "codec-view-prefill":
            from flashcodec_amd import patch_attention as pa
            pa.set_prefill_on_archive(False)
        run(2, 64, 4)                                        # warm-up, same in every run
        one = run(args.c5_batch, args.c5_prompt, args.c5_steps)
        print(json.dumps({"mode": "c5 single run", "kv": args.c5_kv, "batch": args.c5_batch,
                          "prompt": args.c5_prompt, "steps": args.c5_steps, **one}))
        return

    res = {"metric": "end-to-end decode tokens/s (C5)", "unit": "tokens/s", "n_gpus": 1,
           "config": {"workload": "C5 Qwen3-0.6B-shaped greedy decoding", "layers": 28,
                      "hidden": 1024, "q_heads": 16, "kv_heads": 8, "head_dim": 128,
                      "dtype": "bf16", "codec": "jpeg r=8 k=4 int8, materialization-free"
                      + (f", one scale per {args.c5_group} features" if args.c5_group else "")},
           "data": "random-init weights, random prompt ids"}
    run(2, 64, 4)                                              # warm-up (kernels, allocator)
    res["raw_kv_b16"] = run(16, 4096, 256)
    res["raw_kv_b1"] = run(1, 4096, 32)
    fc.apply_flash_codec(model, mode="jpeg", block_size=8, keep_freqs=4, quant_bits=8, **qgroup,
                         materialization_free=True)
    run(2, 64, 4)
    res["codec_b16"] = run(16, 4096, 256)
    res["codec_b1"] = run(1, 4096, 32)
    res["codec_prefill_b16"] = run(16, 4096, 0)
    # the same prefill attending on the reconstructed view (the reference's
    # semantics) instead of the archive
    from flashcodec_amd import patch_attention as pa
    prev = pa.set_prefill_on_archive(False)
    res["codec_view_prefill_b16"] = run(16, 4096, 0)
    pa.set_prefill_on_archive(prev)
    steps = [getattr(m, "_flashcodec_codec_steps", 0) for m in fc.find_attention_modules(model)]
    res["codec_attention_steps_per_layer"] = max(steps) if steps else 0
    res["value"] = res["codec_b16"]["decode_tokens_per_s"]
    res["reference_published_b1_tok_s"] = 40.3
    log(f"bench c5: {res}")
    print(json.dumps(res))


C5_LAYERS, C5_B, C5_HQ, C5_HKV, C5_D = 28, 16, 16, 8, 128


def _c5_codec_cfg(args):
    cfg = dict(mode="jpeg", block_size=8, keep_freqs=4, quant_bits=args.c5_quant_bits)
    if args.c5_group:
        cfg["quant_group"] = args.c5_group
    return cfg


def _c5_codec_name(args):
    if not args.c5_quant_bits:
        return "jpeg r=8 k=4, bf16 coefficients"
    return "jpeg r=8 k=4 int8" + (f", one scale per {args.c5_group} features"
                                  if args.c5_group else "")


def c5step_mode(args):
    """The C5 model's decode-attention step kernel in isolation: 28 layers
    of C5-shaped K/V streams (batch 16, 16 q / 8 kv heads, D=128, bf16, jpeg
    r=8 k=4 int8, --c5-prompt tokens of AR(1) rho=0.95 archived), one decode
    step of every layer (codec_decode_step with the counters on the device:
    token append + in-kernel archive every 8th step + attention, one launch
    per layer) captured as a HIP graph and replayed --steps times, so the
    launches run back to back as in the graph-replayed model.  Algorithmic
    bytes per layer-step: the K and V codes and fp32 scales of the archived
    blocks, the tail rows, the new tokens, q and out."""
    import types
    import torch
    import flashcodec_amd as fc
    from flashcodec_amd import graph
    from flashcodec_amd.cache import FlashCodecLayer
    dev = torch.device("cuda:0")
    cfg = _c5_codec_cfg(args)
    L, B, Hq, Hkv, D = C5_LAYERS, C5_B, C5_HQ, C5_HKV, C5_D
    S0 = args.c5_prompt + 5
    layers = []
    for li in range(L):
        layer = FlashCodecLayer(**cfg)
        for st, seed in ((layer._key_stream, 2 * li + 1), (layer._value_stream, 2 * li + 2)):
            st.append(ar1_device((B, Hkv, S0, D), 0.95, seed, dev).to(torch.bfloat16))
        layers.append(layer)
    torch.cuda.empty_cache()
    steps = args.steps
    cache = types.SimpleNamespace(layers=layers)
    graph.prepare(cache, steps + args.warmup + 2)
    g = torch.Generator(device=dev).manual_seed(7)
    tok = lambda H: torch.randn((B, 1, H, D), generator=g, device=dev).to(torch.bfloat16).transpose(1, 2)
    q_in, k_in, v_in = tok(Hq) / math.sqrt(D), tok(Hkv), tok(Hkv)
    outs = [None] * L

    def one_step():
        for li, layer in enumerate(layers):
            outs[li] = fc.codec_decode_step(q_in, k_in, v_in, layer._key_stream,
                                            layer._value_stream)

    from flashcodec_amd import _native as N
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        one_step()                      # creates the workspace on the capture stream
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    single = N.lib().fc_last_step_single_launch()
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr, stream=stream):
        one_step()
    done = 1
    with torch.cuda.stream(stream):
        for _ in range(args.warmup):
            gr.replay()
    torch.cuda.synchronize()
    done += args.warmup
    nb0 = layers[0]._key_stream.n_blocks + (layers[0]._key_stream._n_raw + done) // 8
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        e0.record(stream)
        for _ in range(steps):
            gr.replay()
        e1.record(stream)
    torch.cuda.synchronize()
    done += steps
    graph.advance_host(cache, done)
    graph.release(cache)
    nb1 = layers[0]._key_stream.n_blocks
    us = e0.elapsed_time(e1) / (steps * L) * 1e3
    ngr = D // 32 if args.c5_group else 1
    nb = (nb0 + nb1) / 2
    # codes + scales (or bf16 coefficients) of the archived blocks, the tail
    # rows (3.5 on average) and the new tokens in bf16, q and out
    row_bytes = D + 4 * ngr if args.c5_quant_bits else 2 * D
    alg = int(2 * B * Hkv * nb * 4 * row_bytes + 2 * B * Hkv * 3.5 * D * 2
              + 2 * B * Hkv * D * 2 + 2 * B * Hq * D * 2)
    res = {"metric": "C5 decode-attention step kernel, us per layer-step", "unit": "us",
           "us_per_layer_step": round(us, 3), "launches_per_layer_step": 1 if single == 1 else None,
           "single_launch": single == 1, "steps": steps, "layers": L,
           "archived_blocks": [nb0, nb1],
           "algorithmic_bytes_per_layer_step": alg, "GBs": round(alg / us / 1e3, 1),
           "hbm_frac": round(alg / us / 1e3 / HBM_PEAK_GBS, 4),
           "config": {"workload": "C5 step kernel", "B": B, "Hq": Hq, "Hkv": Hkv, "D": D,
                      "codec": _c5_codec_name(args), "prompt": args.c5_prompt + 5,
                      "dtype": "bf16"},
           "data": "synthetic AR(1) rho=0.95 K/V, random tokens and queries"}
    log(f"bench c5step: {res}")
    print(json.dumps(res))


def prefill_mode(args):
    """The C5 prefill attention of one layer in isolation: batch 16, 16 q /
    8 kv heads, D=128, bf16, a --c5-prompt-token prompt of AR(1) rho=0.95 K/V
    archived as jpeg r=8 k=4 int8 (--c5-group); codec_prefill_attention (on
    the archive) against the reference's semantics (the reconstructed view
    and PyTorch SDPA, causal)."""
    import torch
    import torch.nn.functional as F
    import flashcodec_amd as fc
    from flashcodec_amd.attention import codec_prefill_attention
    from flashcodec_amd.cache import _CodecStream
    dev = torch.device("cuda:0")
    B, Hq, Hkv, D, S = C5_B, C5_HQ, C5_HKV, C5_D, args.c5_prompt
    if not args.c5_quant_bits:
        print("prefill on the archive takes int8 archives (--c5-quant-bits 8)", file=sys.stderr)
        sys.exit(2)
    cfg = _c5_codec_cfg(args)
    ks, vs = _CodecStream(fc.make_codec(**cfg)), _CodecStream(fc.make_codec(**cfg))
    ks.append(ar1_device((B, Hkv, S, D), 0.95, 1, dev).to(torch.bfloat16))
    vs.append(ar1_device((B, Hkv, S, D), 0.95, 2, dev).to(torch.bfloat16))
    g = torch.Generator(device=dev).manual_seed(3)
    q = (torch.randn((B, Hq, S, D), generator=g, device=dev) / math.sqrt(D)).to(torch.bfloat16)

    def view_sdpa():
        k = ks.read().repeat_interleave(Hq // Hkv, 1)
        v = vs.read().repeat_interleave(Hq // Hkv, 1)
        ks.discard_view()
        vs.discard_view()
        return F.scaled_dot_product_attention(q, k, v, is_causal=True)

    t_arch = timed(lambda: codec_prefill_attention(q, ks, vs), args.steps, args.warmup)
    t_view = timed(view_sdpa, args.steps, args.warmup)
    a = codec_prefill_attention(q, ks, vs).float()
    b = view_sdpa().float()
    flops = 2 * 2 * B * Hq * D * S * (S + 1) / 2
    res = {"metric": "C5 prefill attention of one layer", "unit": "us",
           "archive_us": round(t_arch * 1e3, 1), "view_sdpa_us": round(t_view * 1e3, 1),
           "dense_equivalent_TFLOPs_archive": round(flops / t_arch / 1e9, 1),
           "max_abs_diff_vs_view_sdpa_rel_to_max": float((a - b).abs().max() / b.abs().max()),
           "config": {"workload": "C5 prefill attention, one layer", "B": B, "Hq": Hq, "Hkv": Hkv,
                      "D": D, "S": S, "codec": "jpeg r=8 k=4 int8" + (
                          f", one scale per {args.c5_group} features" if args.c5_group else ""),
                      "dtype": "bf16"},
           "data": "synthetic AR(1) rho=0.95 K/V, q N(0,1)/sqrt(D)"}
    log(f"bench prefill: {res}")
    print(json.dumps(res))



def read_pmc_traffic():
    """HBM bytes per launch of the matrix-core kernel from the committed PMC
    summary (rocprofv3 FETCH_SIZE / WRITE_SIZE of this workload, scaled by
    the copy-kernel calibration), or None when the vector-ALU pass runs or
    no summary exists.  Not measured by this process."""
    from flashcodec_amd import _native as N
    if N.lib().fc_get_attention_pass() == N.PASS_VECTOR or not os.path.exists(PMC_SUMMARY):
        return None
    for line in open(PMC_SUMMARY):
        if line.startswith("traffic_bytes_per_launch:"):
            return int(float(line.split(":", 1)[1]))
    return None


def cpu_baseline(ks, vs, q, min_seconds=10.0):
    """The reference's CPU path on this workload: its torch decode attention
    (oracle/torch_path.py, the restatement of flashcodec/attention.py:101-140
    pinned bit-exact against the reference's outputs) on one sequence at a
    time, dequantising that sequence's int8 rows into the query dtype first
    as the reference does per call; all host cores; sequences taken in turn
    until `min_seconds` have passed.  Host copies of the codes are made
    before the clock starts."""
    import torch
    from oracle import torch_path
    import flashcodec_amd as fc
    cores = len(os.sched_getaffinity(0))
    prev = torch.get_num_threads()
    torch.set_num_threads(cores)
    codes = [st._coeffs[:, :, :NB].cpu() for st in (ks, vs)]
    scales = [st._scales[:, :, :NB].cpu() for st in (ks, vs)]
    raws = [st.raw.cpu() for st in (ks, vs)]
    A = fc.dct_basis(R, K).t()
    qc = q.cpu()

    def one(b):
        sl = slice(b, b + 1)
        rk = torch_path.jpeg_rows(codes[0][sl], scales[0][sl], qc.dtype)
        rv = torch_path.jpeg_rows(codes[1][sl], scales[1][sl], qc.dtype)
        return torch_path.decode_attention(qc[sl], rk, rv, raws[0][sl], raws[1][sl], A,
                                           D ** -0.5)

    one(0)                                        # warm-up
    done = 0
    t0 = time.perf_counter()
    while done < B or time.perf_counter() - t0 < min_seconds:
        one(done % B)
        done += 1
    dt = time.perf_counter() - t0
    torch.set_num_threads(prev)
    seq_bytes = ALG_BYTES_CALL / B
    return {"value": round(done * seq_bytes / dt / 1e9, 3), "unit": "GB/s",
            "cores": cores, "kind": "port",
            "sample": f"{done} sequences of the workload ({done / B:.2f} calls) through the "
                      "reference's torch CPU decode attention (restated in oracle/torch_path.py): "
                      "int8 rows dequantised to fp16, fp16 einsums, fp32 softmax, over 32 q "
                      "heads x (32768 archived + 5 raw tokens)",
            "seconds": round(dt, 3), "cpu_model": cpu_model(),
            "torch_threads": cores}


def check_against_oracle(q, ks, vs, out):
    """Max error of every sequence of `out` against the fp64 oracle,
    relative to max|ref| (the contract's 2e-3 for fp16 outputs)."""
    import numpy as np
    from oracle import oracle as O
    import flashcodec_amd as fc
    nb, r, k = ks.n_blocks, ks.block_size, ks.codec.keep_freqs
    # per-row scales (..., k) or, with quant_group, per-32 scales (..., k, D/32)
    sc = (lambda st: st._scales[:, :, :nb]) if ks.codec.quant_group else \
        (lambda st: st._scales[:, :, :nb, :, 0])
    if ks._scales is None:  # fp coefficients: the rows themselves
        rows = [st._coeffs[:, :, :nb].float().cpu().numpy().astype(np.float64) for st in (ks, vs)]
    else:
        rows = [O.stored_rows_jpeg(st._coeffs[:, :, :nb].cpu().numpy(), sc(st).cpu().numpy())
                for st in (ks, vs)]
    raws = [st.raw.float().cpu().numpy() for st in (ks, vs)]
    A = O.synthesis_matrix("jpeg", r, fc.dct_basis(r, k).numpy())
    ref = O.attention(q[:, :, 0].float().cpu().numpy(), rows[0], rows[1], raws[0], raws[1], A,
                      q.shape[-1] ** -0.5, n_threads=min(16, len(os.sched_getaffinity(0))))
    got = out[:, :, 0].float().cpu().numpy()
    per_seq = np.abs(got - ref).reshape(q.shape[0], -1).max(-1) / np.abs(ref).max()
    return float(per_seq.max()), [float(e) for e in per_seq]


def archive_copy(st):
    """Another stream holding a copy of `st`'s archive and tail (its own
    buffers): one more set for the rotating measurement."""
    from flashcodec_amd.cache import _CodecStream
    c = _CodecStream(st.codec)
    for name in ("_coeffs", "_scales", "_deltas", "_anchors", "_packed", "_packed_mask"):
        t = getattr(st, name, None)
        if t is not None:
            setattr(c, name, t.clone())
    c._capacity, c.n_blocks, c.n_archived = st._capacity, st.n_blocks, st.n_archived
    c.dtype, c.meta = st.dtype, st.meta
    c._adopt_tail(st._raw_buf.clone())
    c._n_raw = st._n_raw
    return c


def c3_mode(args):
    import torch
    import flashcodec_amd as fc
    from flashcodec_amd import _native as N
    from flashcodec_amd.attention import _device_A, _view, launches_per_call
    from flashcodec_amd.cache import _CodecStream

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    log("bench: generating AR(1) K/V and archiving them")
    S = S_ARCH + TAIL
    cfg = dict(mode="jpeg", block_size=R, keep_freqs=K, quant_bits=8)
    ks, vs = _CodecStream(fc.make_codec(**cfg)), _CodecStream(fc.make_codec(**cfg))
    for st, seed in ((ks, 1), (vs, 2)):
        x = ar1_device((B, HKV, S, D), 0.95, seed, dev).to(torch.float16)
        st.append(x)
        del x
    torch.cuda.empty_cache()
    g = torch.Generator(device=dev).manual_seed(3)
    q = (torch.randn((B, HQ, 1, D), generator=g, device=dev) / math.sqrt(D)).to(torch.float16)
    assert ks.n_blocks == NB and ks.raw.shape[-2] == TAIL
    n_sets = max(1, args.sets)
    sets = [(ks, vs)] + [(archive_copy(ks), archive_copy(vs)) for _ in range(n_sets - 1)]

    L = N.lib()
    n_splits = args.splits or L.fc_attention_splits(N.STORE_JPEG_I8, N.F16, N.F16, K, NB, B, HKV,
                                                    HQ // HKV, D, N.num_cus(dev))
    keep = []
    A = _device_A(ks.codec, R, dev)
    out_c = torch.empty_like(q)
    # zero-filled once: its counters return to zero after every call
    ws = torch.zeros(L.fc_attention_workspace_bytes(B, HQ, D, n_splits), dtype=torch.uint8,
                     device=dev)

    def abi_args(kst, vst):
        return (q.data_ptr(), N.F16, q.stride(0), q.stride(1), B, HQ, HKV, D, N.STORE_JPEG_I8,
                N.F16, R, K, NB, _view(kst, keep), _view(vst, keep), TAIL, A.data_ptr(),
                D ** -0.5, out_c.data_ptr(), out_c.stride(0), out_c.stride(1), ws.data_ptr(),
                n_splits, N.stream_ptr(dev))
    set_args = [abi_args(*kv) for kv in sets]

    if args.splits:
        def call(i):
            N.check(L.fc_decode_attention(*set_args[i % n_sets]), "fc_decode_attention")
            return out_c
    else:
        def call(i):
            kst, vst = sets[i % n_sets]
            return fc.codec_decode_attention(q, kst, vst)

    def events_ms(fn, steps, stream=None):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for i in range(steps):
            fn(i)
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / steps

    n_settle = settle(call)
    log(f"bench: settle {n_settle} calls, warmup {args.warmup}, steps {args.steps}, "
        f"splits {n_splits}, sets {n_sets}")
    for i in range(args.warmup):
        call(i)
    torch.cuda.synchronize()
    ms = events_ms(call, args.steps)
    log(f"bench: {ms * 1e3:.1f} us per call over {n_sets} archive sets")

    # dominant kernel: the call is one launch of the split kernel (its last
    # workgroup per head group merges); back-to-back launches through the C
    # ABI, cycling over the sets, between two events on the stream they are
    # launched on (the stream N.stream_ptr hands the library)
    stream = torch.cuda.current_stream(dev)

    def launch(i):
        N.check(L.fc_decode_attention(*set_args[i % n_sets]), "fc_decode_attention")

    for i in range(2 * n_sets):
        launch(i)
    torch.cuda.synchronize()
    launch_ms = events_ms(launch, args.steps, stream)
    achieved = ALG_BYTES_CALL / (launch_ms * 1e-3) / 1e9
    log(f"bench: kernel {launch_ms * 1e3:.1f} us per launch, {achieved:.0f} GB/s")
    single_ms = events_ms(lambda i: N.check(L.fc_decode_attention(*set_args[0]), "attn"),
                          args.steps, stream)
    single = ALG_BYTES_CALL / (single_ms * 1e-3) / 1e9
    log(f"bench: one repeated set {single_ms * 1e3:.1f} us per launch, {single:.0f} GB/s")

    out = fc.codec_decode_attention(q, ks, vs)
    err, per_seq = check_against_oracle(q, ks, vs, out)
    log(f"bench: max error vs the fp64 oracle over all {B} sequences {err:.2e}")
    lpc = launches_per_call(N.STORE_JPEG_I8, n_splits)
    result = {
        "metric": METRIC,
        "value": round(ALG_BYTES_CALL / (ms * 1e-3) / 1e9, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "settle": {"calls": n_settle, "min_seconds": SETTLE_S,
                   "note": "untimed calls before the warm-up steps: the device runs a new "
                           "load below its steady rate for its first milliseconds"},
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "accumulate": "f32",
        "data": "synthetic AR(1) rho=0.95 K/V (fp16, archived int8 by the kernels), "
                "q fp16 N(0,1)/sqrt(D)",
        "config": {"workload": "C3 coefficient-domain split-K decode attention",
                   "B": B, "Hq": HQ, "Hkv": HKV, "D": D, "S_archived": S_ARCH, "raw_tail": TAIL,
                   "block": R, "keep_freqs": K, "coeffs": "int8 + fp32 scales",
                   "q_dtype": "fp16", "n_splits": n_splits, "archive_sets": n_sets,
                   "algorithmic_bytes_per_call": ALG_BYTES_CALL},
        "hbm_frac": round(ALG_BYTES_CALL / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "tokens_per_s": round(B / (ms * 1e-3), 1),
        "launches_per_call": lpc,
        "roofline": {"bound": "hbm", "kernel": split_kernel_name(n_splits),
                     "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": read_pmc_traffic(),
                     "traffic_source": "committed rocprofv3 FETCH_SIZE/WRITE_SIZE summary "
                                       "(profiles/attn_split_c3_pmc.md), not this run",
                     "algorithmic_bytes_per_launch": ALG_BYTES_CALL,
                     "avg_launch_us": round(launch_ms * 1e3, 2),
                     "archive_sets": n_sets},
        "single_set": {"avg_launch_us": round(single_ms * 1e3, 2), "achieved": round(single, 2),
                       "frac": round(single / HBM_PEAK_GBS, 4),
                       "note": "the same launches repeated on one archive set, which the "
                               "256 MB last-level cache partly serves"},
        "check": {"vs_oracle_max_rel_err": err, "per_sequence": per_seq, "tolerance": 2e-3,
                  "sequences": B},
    }
    if not args.no_cpu_baseline:
        log("bench: cpu baseline (the reference's torch CPU path, >= 10 s of the workload)")
        result["cpu_baseline"] = cpu_baseline(ks, vs, q)
    else:
        result["cpu_baseline"] = None
    print(json.dumps(result))
    if not err <= 2e-3:
        log(f"bench: output differs from the oracle beyond the tolerance ({err:.2e} > 2e-3)")
        sys.exit(3)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=400)
    ap.add_argument("--warmup", type=int, default=40)
    ap.add_argument("--mode", choices=["c3", "c1", "c2", "c4", "c5", "c5step", "prefill", "refshapes",
                                       "shapes", "copy"],
                    default="c3")
    ap.add_argument("--copy-bytes", type=int, default=1 << 30)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--sets", type=int, default=4,
                    help="c3: archive copies the timed calls cycle over (1: one repeated set)")
    ap.add_argument("--splits", type=int, default=0, help="override the split count")
    ap.add_argument("--c5-steps", type=int, default=None,
                    help="c5: one run of this many decode steps (0: prefill only)")
    ap.add_argument("--c5-batch", type=int, default=16)
    ap.add_argument("--c5-prompt", type=int, default=4096)
    ap.add_argument("--c5-kv", choices=["raw", "codec", "codec-view-prefill"], default="codec")
    ap.add_argument("--c5-group", type=int, choices=[0, 32], default=0,
                    help="C5 codec quantizer group (32: one scale per 32 features)")
    ap.add_argument("--c5-quant-bits", type=int, choices=[0, 8], default=8,
                    help="c5step: 0 stores the bf16 coefficients (the reference's default codec)")
    ap.add_argument("--c5-graph", action="store_true",
                    help="c5: codec decode steps replayed from a captured HIP graph")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (--gpus {args.gpus} "
              "requested); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        sys.exit(2)
    if args.mode == "copy":
        return copy_mode(args)
    if args.mode == "c1":
        return c1_mode(args)
    if args.mode == "c2":
        return c2_mode(args)
    if args.mode == "refshapes":
        return refshapes_mode(args)
    if args.mode == "shapes":
        return shapes_mode(args)
    if args.mode == "c5":
        return c5_mode(args)
    if args.mode == "c5step":
        return c5step_mode(args)
    if args.mode == "prefill":
        return prefill_mode(args)
    if args.mode == "c4":
        return c4_mode(args)

    return c3_mode(args)

if __name__ == "__main__":
    main()
