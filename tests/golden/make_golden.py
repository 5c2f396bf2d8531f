"""Write the golden vectors of the KV-codec hot path from the reference.

Run in the build container only (the reference is not present on GPU
boxes):  python tests/golden/make_golden.py  [--ref /root/reference]

The reference (flashcodec-kv 1.0.0, pure Python on PyTorch's CPU kernels) is
imported to record input/output vectors of exactly the functions whose bits
no closed form pins:
  * dct_basis bits (torch's CPU cos is not correctly rounded),
  * dct_compress / dct_decompress rounding (the CPU GEMM's order),
  * quantize_coeffs codes and scale bits,
  * png_filter Top-M survivors under ties (torch's CPU topk order),
  * png_reconstruct rounding (CPU cumsum accumulates in double),
  * _CodecStream.append/read/crop end to end (cat + slice + archive path),
  * the torch-path decode attention (tolerance reference only).
Inputs are generated here with numpy PCG64; bf16 tensors are stored as
uint16 bit patterns, everything in tests/golden/*.npz with a JSON manifest.
"""

import argparse
import json
import math
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))

TORCH_DT = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}


def store(t):
    """torch tensor -> numpy storage array (bf16 as uint16 bits)."""
    t = t.detach().cpu().contiguous()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def make_input(shape, dtype, seed, kind="ar1", rho=0.95, scaled=False):
    rng = np.random.Generator(np.random.PCG64(seed))
    *lead, S, D = shape
    if kind == "ar1":
        eps = rng.standard_normal(tuple(lead) + (S, D))
        x = np.empty_like(eps)
        x[..., 0, :] = eps[..., 0, :]
        c = math.sqrt(1 - rho * rho)
        for t in range(1, S):
            x[..., t, :] = rho * x[..., t - 1, :] + c * eps[..., t, :]
    elif kind == "ties":
        # small integers / 8: exact ties of |delta| are frequent
        x = rng.integers(-6, 7, size=tuple(lead) + (S, D)) / 8.0
    elif kind == "randn":
        x = rng.standard_normal(tuple(lead) + (S, D))
    else:
        raise ValueError(kind)
    if scaled:
        sc = np.exp(rng.uniform(math.log(0.1), math.log(10.0), size=tuple(lead) + (1, D)))
        x = x * sc
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(TORCH_DT[dtype])


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--ref", default="/root/reference")
    args = ap.parse_args()
    sys.path.insert(0, args.ref)
    import flashcodec as F  # the reference
    from flashcodec.attention import codec_decode_attention
    from flashcodec.cache import _CodecStream, make_codec

    torch.manual_seed(0)
    manifest = {"reference": f"flashcodec {F.__version__}", "torch": torch.__version__}

    # ---------------------------------------------------------------- basis
    basis = {}
    for r in (2, 4, 8, 12, 16, 32, 64):
        full = F.dct_basis(r, r)
        for k in range(1, r + 1):
            assert torch.equal(F.dct_basis(r, k), full[:k])
        basis[f"r{r}"] = store(full)
    np.savez_compressed(os.path.join(HERE, "basis.npz"), **basis)
    manifest["basis"] = sorted(basis)

    # ---------------------------------------------------------------- jpeg
    jpeg_cases = [
        # name, dtype, r, k, shape, kind, scaled
        ("f32_r8k2", "f32", 8, 2, (2, 3, 64, 40), "ar1", False),
        ("f16_r8k4", "f16", 8, 4, (2, 3, 61, 128), "ar1", True),
        ("bf16_r8k4", "bf16", 8, 4, (1, 4, 64, 64), "ar1", True),
        ("f32_r16k4", "f32", 16, 4, (1, 2, 96, 32), "randn", False),
        ("f16_r4k1", "f16", 4, 1, (2, 2, 30, 16), "ar1", False),
        ("f32_r8k8", "f32", 8, 8, (1, 2, 48, 24), "randn", True),
        ("f32_r12k3", "f32", 12, 3, (1, 2, 40, 24), "ar1", False),
        ("bf16_r32k4", "bf16", 32, 4, (1, 2, 64, 32), "ar1", True),
        ("f16_r16k16", "f16", 16, 16, (1, 1, 32, 8), "randn", False),
    ]
    jpeg = {}
    meta = {}
    for i, (name, dt, r, k, shape, kind, scaled) in enumerate(jpeg_cases):
        x = make_input(shape, dt, 100 + i, kind, scaled=scaled)
        if name == "f16_r8k4":
            x[0, 0, 8:16] = 0                   # an all-zero block: scale 1
            x[0, 1, 16:24] = x[0, 1, 16:24] * 1e-6  # subnormal-range scales
        coef = F.dct_compress(x, r, k)
        q, s = F.quantize_coeffs(coef)
        jpeg[f"{name}/x"] = store(x)
        jpeg[f"{name}/coef"] = store(coef)
        jpeg[f"{name}/codes"] = store(q)
        jpeg[f"{name}/scales"] = store(s[..., 0])
        jpeg[f"{name}/deq_f32"] = store(F.dequantize_coeffs(q, s))
        jpeg[f"{name}/deq_T"] = store(F.dequantize_coeffs(q, s, TORCH_DT[dt]))
        S = shape[-2]
        jpeg[f"{name}/rec"] = store(F.dct_decompress(coef, r, out_len=S))
        jpeg[f"{name}/rec_q"] = store(F.dct_decompress(F.dequantize_coeffs(q, s), r, out_len=S))
        meta[name] = dict(dtype=dt, r=r, k=k, shape=list(shape))
    np.savez_compressed(os.path.join(HERE, "jpeg.npz"), **jpeg)
    manifest["jpeg"] = meta

    # ---------------------------------------------------------------- png
    png_cases = [
        ("f32_r8_k1", "f32", 8, 1.0, (2, 3, 64, 40), "ar1"),
        ("f32_r8_k05", "f32", 8, 0.5, (2, 3, 61, 40), "ar1"),
        ("f32_r16_k025", "f32", 16, 0.25, (1, 2, 128, 32), "ar1"),
        ("f32_r16_k01", "f32", 16, 0.1, (1, 2, 64, 32), "randn"),
        ("f16_r16_k025_ties", "f16", 16, 0.25, (2, 2, 64, 64), "ties"),
        ("bf16_r8_k05_ties", "bf16", 8, 0.5, (2, 2, 64, 32), "ties"),
        ("f32_r8_k025_ties", "f32", 8, 0.25, (2, 4, 64, 64), "ties"),
        ("bf16_r8_k1", "bf16", 8, 1.0, (1, 2, 40, 128), "randn"),
        ("f32_r4_k05", "f32", 4, 0.5, (1, 2, 30, 16), "ties"),
        ("f16_r32_k025_ties", "f16", 32, 0.25, (1, 1, 64, 16), "ties"),
    ]
    png = {}
    meta = {}
    for i, (name, dt, r, keep, shape, kind) in enumerate(png_cases):
        x = make_input(shape, dt, 200 + i, kind)
        d, a = F.png_filter(x, r, keep)
        png[f"{name}/x"] = store(x)
        png[f"{name}/deltas"] = store(d)
        png[f"{name}/anchors"] = store(a)
        png[f"{name}/rec"] = store(F.png_reconstruct(d, a))
        meta[name] = dict(dtype=dt, r=r, keep=keep, shape=list(shape))
    np.savez_compressed(os.path.join(HERE, "png.npz"), **png)
    manifest["png"] = meta

    # ---------------------------------------------------------------- streams
    stream_cases = [
        # name, cfg, dtype, shape (B,H,S,D), feed ("token" | "bulk" | chunk size)
        ("jpeg_i8_f16_token", dict(mode="jpeg", block_size=8, keep_freqs=4, quant_bits=8),
         "f16", (2, 2, 43, 64), "token"),
        ("jpeg_i8_f16_bulk", dict(mode="jpeg", block_size=8, keep_freqs=4, quant_bits=8),
         "f16", (2, 2, 43, 64), "bulk"),
        ("jpeg_f32_token", dict(mode="jpeg", block_size=8, keep_freqs=2), "f32",
         (1, 3, 37, 32), "token"),
        ("png_bf16_k05_chunk5", dict(mode="png", block_size=8, keep_ratio=0.5), "bf16",
         (2, 2, 45, 32), 5),
        ("png_f32_k1_token", dict(mode="png", block_size=16, keep_ratio=1.0), "f32",
         (1, 2, 50, 32), "token"),
        ("jpeg_i8_bf16_chunk3", dict(mode="jpeg", block_size=8, keep_freqs=2, quant_bits=8),
         "bf16", (1, 2, 40, 128), 3),
    ]
    st = {}
    meta = {}
    for i, (name, cfg, dt, shape, feed) in enumerate(stream_cases):
        x = make_input(shape, dt, 300 + i, "ar1", scaled=True)
        s = _CodecStream(make_codec(**cfg))
        S = shape[-2]
        if feed == "bulk":
            s.append(x)
        else:
            step = 1 if feed == "token" else int(feed)
            for t in range(0, S, step):
                s.append(x[..., t:t + step, :])
        st[f"{name}/x"] = store(x)
        n = s.n_blocks
        if s.codec.name == "jpeg":
            st[f"{name}/coeffs"] = store(s._coeffs[:, :, :n])
            if s.codec.quantized:
                st[f"{name}/scales"] = store(s._scales[:, :, :n, :, 0])
        else:
            st[f"{name}/deltas"] = store(s._deltas[:, :, :n])
            st[f"{name}/anchors"] = store(s._anchors[:, :, :n])
        st[f"{name}/read"] = store(s.read())
        s.crop(-5)
        st[f"{name}/read_crop5"] = store(s.read())
        meta[name] = dict(cfg=cfg, dtype=dt, shape=list(shape), feed=feed, n_blocks=n,
                          capacity=0)
    np.savez_compressed(os.path.join(HERE, "stream.npz"), **st)
    manifest["stream"] = meta

    # ---------------------------------------------------------------- attention
    attn_cases = [
        ("jpeg_i8_f32_g2_t3", dict(mode="jpeg", block_size=8, keep_freqs=2, quant_bits=8),
         "f32", 2, 4, 8 * 12 + 3, 32),
        ("jpeg_f32_k8_g1_t0", dict(mode="jpeg", block_size=8, keep_freqs=8), "f32", 1, 2, 96, 32),
        ("png_f32_k1_g4_t5", dict(mode="png", block_size=8, keep_ratio=1.0), "f32", 4, 2,
         8 * 10 + 5, 32),
        ("png_f32_k05_g2_t7", dict(mode="png", block_size=16, keep_ratio=0.5), "f32", 2, 2,
         16 * 5 + 7, 64),
        ("jpeg_i8_f16_g4_t5", dict(mode="jpeg", block_size=8, keep_freqs=4, quant_bits=8),
         "f16", 4, 2, 8 * 16 + 5, 128),
    ]
    at = {}
    meta = {}
    for i, (name, cfg, dt, G, Hk, S, D) in enumerate(attn_cases):
        B = 2
        k = make_input((B, Hk, S, D), dt, 400 + i, "ar1", scaled=True)
        v = make_input((B, Hk, S, D), dt, 450 + i, "ar1", scaled=True)
        rng = np.random.Generator(np.random.PCG64(500 + i))
        q = torch.from_numpy((rng.standard_normal((B, Hk * G, 1, D)) / math.sqrt(D))
                             .astype(np.float32)).to(TORCH_DT[dt])
        ks, vs = _CodecStream(make_codec(**cfg)), _CodecStream(make_codec(**cfg))
        ks.append(k)
        vs.append(v)
        out = codec_decode_attention(q, ks, vs, impl="torch")
        at[f"{name}/k"] = store(k)
        at[f"{name}/v"] = store(v)
        at[f"{name}/q"] = store(q)
        at[f"{name}/out"] = store(out)
        meta[name] = dict(cfg=cfg, dtype=dt, G=G, Hk=Hk, S=S, D=D, B=B)
    np.savez_compressed(os.path.join(HERE, "attention.npz"), **at)
    manifest["attention"] = meta

    with open(os.path.join(HERE, "manifest.json"), "w") as fh:
        json.dump(manifest, fh, indent=1, sort_keys=True)
    sizes = {f: os.path.getsize(os.path.join(HERE, f)) for f in os.listdir(HERE)
             if f.endswith(".npz")}
    print("wrote", sizes)


if __name__ == "__main__":
    main()
