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
The roofline object covers that kernel, each launch timed with HIP events on
the stream it is launched on.  `cpu_baseline` times the fp64 CPU oracle on
the same workload's sequences for at least 10 s (one whole call or more).

  python bench.py [--steps K] [--warmup W] [--gpus 1]
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


def split_kernel_name():
    """Kernel of this workload's call (int8 codes, fp16 q, D=128, 4 rows per
    block, groups of 4 q heads): the matrix-core split pass with its merge
    fused in (one launch)."""
    if os.environ.get("FLASHCODEC_AMD_ATTN", "").startswith("v"):
        return "attn_split_kernel + attn_merge_head_kernel"
    return "attn_split_i8_mfma<4,4,4> (merge fused)"


def read_pmc_traffic():
    """HBM bytes per launch of the matrix-core kernel from the committed PMC
    summary, if any (None for the vector-ALU variant, which it does not cover)."""
    if os.environ.get("FLASHCODEC_AMD_ATTN", "").startswith("v") or not os.path.exists(PMC_SUMMARY):
        return None
    for line in open(PMC_SUMMARY):
        if line.startswith("traffic_bytes_per_launch:"):
            return int(float(line.split(":", 1)[1]))
    return None


def cpu_baseline(q, ks, vs, min_seconds=10.0):
    """The CPU restatement of the path (oracle/) on the same workload: per
    sequence, dequantise the int8 K/V codes to rows and run fp64 decode
    attention over 32 q heads.  Sequences are taken in turn until at least
    `min_seconds` have passed and every sequence has run once (one whole
    call); host copies of the codes are made before the clock starts.
    Returns (sequence-0 output, baseline record)."""
    import numpy as np
    from oracle import oracle as O
    import flashcodec_amd as fc
    threads = min(len(os.sched_getaffinity(0)), 16)
    codes = [st._coeffs[:, :, :NB].cpu().numpy() for st in (ks, vs)]
    scales = [st._scales[:, :, :NB, :, 0].cpu().numpy() for st in (ks, vs)]
    raws = [st.raw.float().cpu().numpy() for st in (ks, vs)]
    A = O.synthesis_matrix("jpeg", R, fc.dct_basis(R, K).numpy())
    qn = q[:, :, 0].float().cpu().numpy()

    def one(b):
        rk = O.stored_rows_jpeg(codes[0][b:b + 1], scales[0][b:b + 1])
        rv = O.stored_rows_jpeg(codes[1][b:b + 1], scales[1][b:b + 1])
        return O.attention(qn[b:b + 1], rk, rv, raws[0][b:b + 1], raws[1][b:b + 1], A,
                           D ** -0.5, n_threads=threads)

    ref0, done = None, 0
    t0 = time.perf_counter()
    while done < B or time.perf_counter() - t0 < min_seconds:
        o = one(done % B)
        if done == 0:
            ref0 = o
        done += 1
    dt = time.perf_counter() - t0
    seq_bytes = ALG_BYTES_CALL / B
    return ref0, {"value": round(done * seq_bytes / dt / 1e9, 3), "unit": "GB/s",
                  "cores": threads, "kind": "port",
                  "sample": f"{done} sequences of the workload ({done / B:.2f} calls): int8 "
                            "codes -> fp64 rows (numpy) -> fp64 decode attention over 32 q "
                            "heads x (32768 archived + 5 raw tokens) (C++ oracle, OpenMP)",
                  "seconds": round(dt, 3)}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--mode", choices=["c3", "copy"], default="c3")
    ap.add_argument("--copy-bytes", type=int, default=1 << 30)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--splits", type=int, default=0, help="override the split count")
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

    import numpy as np
    import flashcodec_amd as fc
    from flashcodec_amd import _native as N
    from flashcodec_amd.attention import _device_A, _view
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

    L = N.lib()
    n_splits = args.splits or L.fc_attention_default_splits(NB, B, HKV, HQ // HKV, N.num_cus(dev))
    keep = []
    kv, vv = _view(ks, keep), _view(vs, keep)
    A = _device_A(ks.codec, R, dev)
    out_c = torch.empty_like(q)
    # zero-filled once: its arrival counters return to zero after every call
    ws = torch.zeros(L.fc_attention_workspace_bytes(B, HQ, D, n_splits), dtype=torch.uint8,
                     device=dev)
    abi_args = (q.data_ptr(), N.F16, q.stride(0), q.stride(1), B, HQ, HKV, D, N.STORE_JPEG_I8,
                N.F16, R, K, NB, kv, vv, TAIL, A.data_ptr(), D ** -0.5, out_c.data_ptr(),
                out_c.stride(0), out_c.stride(1), ws.data_ptr(), n_splits, N.stream_ptr(dev))

    if args.splits:
        def call():
            N.check(L.fc_decode_attention(*abi_args), "fc_decode_attention")
            return out_c
    else:
        def call():
            return fc.codec_decode_attention(q, ks, vs)

    log(f"bench: warmup {args.warmup}, steps {args.steps}, splits {n_splits}")
    for _ in range(args.warmup):
        out = call()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(args.steps):
        out = call()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / args.steps
    log(f"bench: {ms * 1e3:.1f} us per call")

    # dominant kernel: the call is one launch of the split kernel (its last
    # workgroup per head group merges); K back-to-back launches through the
    # C ABI between two events on the stream they are launched on
    for _ in range(3):
        N.check(L.fc_decode_attention(*abi_args), "fc_decode_attention")
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(dev)   # the stream N.stream_ptr hands the library
    k0, k1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    k0.record(stream)
    for _ in range(args.steps):
        N.check(L.fc_decode_attention(*abi_args), "fc_decode_attention")
    k1.record(stream)
    torch.cuda.synchronize()
    launch_ms = k0.elapsed_time(k1) / args.steps
    achieved = ALG_BYTES_CALL / (launch_ms * 1e-3) / 1e9
    log(f"bench: kernel {launch_ms * 1e3:.1f} us per launch, {achieved:.0f} GB/s")

    result = {
        "metric": METRIC,
        "value": round(ALG_BYTES_CALL / (ms * 1e-3) / 1e9, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
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
                   "q_dtype": "fp16", "n_splits": n_splits,
                   "algorithmic_bytes_per_call": ALG_BYTES_CALL},
        "hbm_frac": round(ALG_BYTES_CALL / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "tokens_per_s": round(B / (ms * 1e-3), 1),
        "launches_per_call": 1,
        "roofline": {"bound": "hbm", "kernel": split_kernel_name(),
                     "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": read_pmc_traffic(),
                     "algorithmic_bytes_per_launch": ALG_BYTES_CALL,
                     "avg_launch_us": round(launch_ms * 1e3, 2)},
    }
    if not args.no_cpu_baseline:
        log("bench: cpu baseline (fp64 oracle, >= 10 s of the workload)")
        ref, cpu = cpu_baseline(q, ks, vs)
        got = out[:1, :, 0].float().cpu().numpy()
        err = float(np.abs(got - ref).max() / np.abs(ref).max())
        result["cpu_baseline"] = cpu
        result["check"] = {"vs_oracle_max_rel_err_seq0": err, "tolerance": 2e-3}
    else:
        result["cpu_baseline"] = None
    print(json.dumps(result))


if __name__ == "__main__":
    main()
