"""GPU: reconstruct-free causal prefill attention on int8 jpeg archives
(fc_prefill_attention) against fp64 causal attention over the codec's exact
reconstruction, and the patched HF prefill that uses it.

The oracle is the coefficient-domain definition the decode oracle uses:
stored rows (codes x scales) in fp64 synthesised through the codec's A
matrix, raw-tail tokens as stored, brute-force fp64 softmax(q K^T * scale +
causal mask) V.  The reference's prefill attends on the read() view, whose
tokens are that reconstruction rounded to the stream dtype; in bf16 that
rounding alone moves the attention by up to ~2.2e-3 of max|out|
(measured), so the view is not the oracle.  Tolerance: the contract's 2e-3
of max|ref| plus half an ulp of the output dtype.
"""

import math

import numpy as np
import pytest
import torch

import flashcodec_amd as fc
from flashcodec_amd.attention import codec_prefill_attention
from flashcodec_amd.cache import _CodecStream
from tests.conftest import to_values, torch_dtype
from tests.test_gpu_attention import HALF_ULP

pytestmark = pytest.mark.gpu
DEV = "cuda"


def view_oracle(oracle, st):
    """The stream's tokens (B, H, S, D) in fp64: the archive's stored rows
    (oracle.stored_rows_jpeg) synthesised through A, then the raw tail."""
    n, r, k = st.n_blocks, st.block_size, st.codec.keep_freqs
    parts = []
    if n:
        sc = st._scales[:, :, :n] if st.codec.quant_group else st._scales[:, :, :n, :, 0]
        rows = oracle.stored_rows_jpeg(st._coeffs[:, :, :n].cpu().numpy(), sc.cpu().numpy())
        A = oracle.synthesis_matrix("jpeg", r, fc.dct_basis(r, k).numpy())
        B, H, _, _, D = rows.shape
        parts.append(np.einsum("ps,bhnsd->bhnpd", A, rows).reshape(B, H, n * r, D))
    if st.raw is not None:
        parts.append(to_values(st.raw).astype(np.float64))
    return np.concatenate(parts, axis=2)


def causal_reference(q, kview, vview, P0, scale, rows=None):
    """fp64 causal attention of queries at positions P0 + i (q (B, Hq, Sq,
    D) values) over the views (B, Hkv, S, D); `rows` limits the checked
    query indices."""
    B, Hq, Sq, D = q.shape
    G = Hq // kview.shape[1]
    rows = range(Sq) if rows is None else rows
    out = np.zeros((B, Hq, len(rows), D))
    for n, i in enumerate(rows):
        L = P0 + i + 1
        for h in range(Hq):
            kk, vv = kview[:, h // G, :L], vview[:, h // G, :L]
            s = np.einsum("bd,btd->bt", q[:, h, i].astype(np.float64), kk) * scale
            p = np.exp(s - s.max(-1, keepdims=True))
            p /= p.sum(-1, keepdims=True)
            out[:, h, n] = np.einsum("bt,btd->bd", p, vv)
    return out


def check(out, ref, dt):
    err = np.abs(out - ref)
    tol = 2e-3 * np.abs(ref).max() + HALF_ULP[dt] * np.abs(ref)
    assert not (err > tol).any(), f"max err {err.max():.3e} vs max|ref| {np.abs(ref).max():.3e}"


def streams(dt, B, Hkv, S, D, k, seed, oracle, group=0, r=8):
    cfg = dict(mode="jpeg", block_size=r, keep_freqs=k, quant_bits=8)
    if group:
        cfg["quant_group"] = group
    x = [torch.from_numpy(oracle.ar1((B, Hkv, S, D), 0.9, seed + i)).to(torch_dtype(dt)).to(DEV)
         for i in range(2)]
    ks, vs = _CodecStream(fc.make_codec(**cfg)), _CodecStream(fc.make_codec(**cfg))
    return ks, vs, x


CASES = [
    # dt, B, Hkv, G, D, k, S (prompt), S0 (tokens cached before it)
    ("bf16", 2, 2, 2, 128, 4, 8 * 37 + 5, 0),
    ("f16", 1, 2, 4, 128, 4, 8 * 20 + 3, 0),
    ("bf16", 1, 1, 1, 64, 2, 8 * 30 + 7, 0),
    ("f16", 2, 2, 3, 64, 1, 8 * 12 + 1, 0),
    ("bf16", 1, 2, 8, 256, 4, 8 * 9 + 2, 0),
    ("f16", 1, 1, 16, 128, 2, 8 * 11, 0),
    ("bf16", 2, 2, 2, 128, 4, 77, 8 * 25 + 3),       # chunked: 203 cached, 77 more
    ("f16", 1, 2, 2, 128, 4, 5, 0),                  # shorter than a block: tail only
    ("bf16", 1, 2, 2, 128, 4, 3, 8 * 10 + 6),         # 3 more tokens completing a block
    # per-32 scales (quant_group=32)
    ("bf16", 2, 2, 2, 128, 4, 8 * 37 + 5, 0, 32),
    ("f16", 1, 1, 16, 128, 2, 8 * 11, 0, 32),
    ("f16", 2, 2, 3, 64, 1, 8 * 12 + 1, 0, 32),
    ("bf16", 1, 2, 8, 256, 4, 8 * 9 + 2, 0, 32),
    ("bf16", 2, 2, 2, 128, 4, 77, 8 * 25 + 3, 32),
    # other block sizes (the last field): r = 4 (s == r), 16 (the unrolled
    # tap loop's limit) and 32 (the tap loop that is not unrolled), with
    # chunked and tail-only prefills
    ("bf16", 1, 2, 2, 128, 4, 4 * 50 + 3, 0, 0, 4),
    ("f16", 2, 1, 4, 64, 2, 4 * 9 + 1, 4 * 30 + 2, 0, 4),
    ("f16", 2, 2, 4, 128, 2, 16 * 20 + 9, 0, 0, 16),
    ("bf16", 1, 2, 2, 128, 4, 45, 16 * 12 + 5, 0, 16),
    ("bf16", 1, 2, 8, 256, 1, 16 * 6 + 15, 0, 32, 16),
    ("bf16", 1, 2, 2, 64, 4, 32 * 10 + 17, 0, 0, 32),
    ("f16", 1, 2, 2, 128, 4, 20, 0, 0, 32),
    ("f16", 1, 1, 4, 128, 1, 50, 32 * 6 + 30, 0, 32),
    ("bf16", 2, 2, 2, 128, 2, 32 * 5 + 31, 0, 32, 32),
    # the workgroup-shared pass (4 stored rows, one scale per row, D = 64 /
    # 128, r = 4 / 8) at D = 64 and with 1 and 16 query heads per kv head
    # (16 and 1 tokens per wavefront); r = 16 at D = 64 (register pass)
    ("f16", 2, 2, 2, 64, 4, 8 * 25 + 5, 0),
    ("bf16", 1, 2, 4, 64, 4, 4 * 41 + 2, 4 * 7 + 1, 0, 4),
    ("f16", 1, 1, 2, 64, 4, 16 * 13 + 11, 0, 0, 16),
    ("bf16", 1, 2, 1, 128, 4, 8 * 33 + 7, 0),
    ("f16", 1, 1, 16, 128, 4, 8 * 11 + 3, 8 * 6),
]


def _case_id(c):
    return (f"{c[0]}-G{c[3]}-D{c[4]}-k{c[5]}-S{c[6]}+{c[7]}"
            + (f"-g{c[8]}" if len(c) > 8 and c[8] else "")
            + (f"-r{c[9]}" if len(c) > 9 else ""))


@pytest.mark.parametrize("case", CASES, ids=[_case_id(c) for c in CASES])
def test_prefill_matches_causal_attention_on_the_view(case, oracle):
    _prefill_case(case, oracle)


def _draw_prefill(seed, n):
    """Seeded random prefill cases (same list on every run): dtype, batch,
    kv heads, query heads per kv head, head size, kept frequencies, prompt
    and cached lengths (chunked prefills, tails, prompts shorter than a
    block), scale layout and block size."""
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        r = int(rng.choice([4, 8, 16, 32]))
        k = int(rng.choice([kk for kk in (1, 2, 4) if kk <= r]))
        D = int(rng.choice([64, 128, 256]))
        G = int(rng.choice([1, 2, 3, 4, 8, 16]))
        S = int(rng.integers(1, 320))
        S0 = int(rng.choice([0, 0, int(rng.integers(1, 200))]))
        out.append((str(rng.choice(["f16", "bf16"])), int(rng.integers(1, 3)),
                    int(rng.choice([1, 2])), G, D, k, S, S0, int(rng.choice([0, 32])), r))
    return out


SWEEP = _draw_prefill(2030, 24)


@pytest.mark.parametrize("case", SWEEP, ids=[f"p{i}" for i in range(len(SWEEP))])
def test_prefill_sweep(case, oracle):
    _prefill_case(case, oracle)


def _prefill_case(case, oracle):
    dt, B, Hkv, G, D, k, S, S0 = case[:8]
    group = case[8] if len(case) > 8 else 0
    r = case[9] if len(case) > 9 else 8
    print(f"case prefill {case}", flush=True)
    ks, vs, (kx, vx) = streams(dt, B, Hkv, S0 + S, D, k, 40 + G + D + S, oracle, group, r)
    if S0:
        ks.append(kx[:, :, :S0])
        vs.append(vx[:, :, :S0])
    ks.append(kx[:, :, S0:])
    vs.append(vx[:, :, S0:])
    rng = np.random.default_rng(41)
    qn = (rng.standard_normal((B, Hkv * G, S, D)) / math.sqrt(D)).astype(np.float32)
    qn[:, :, :, :3] *= 6.0                      # a few larger features, as real queries have
    q = torch.from_numpy(qn).to(torch_dtype(dt)).to(DEV)
    out = codec_prefill_attention(q, ks, vs)
    assert out.shape == q.shape and out.dtype == q.dtype
    assert ks._rec is None and vs._rec is None
    ref = causal_reference(to_values(q), view_oracle(oracle, ks), view_oracle(oracle, vs), S0,
                           D ** -0.5)
    check(to_values(out), ref, dt)


def test_prefill_c5_prompt_shape(oracle):
    """One sequence of the C5 prefill: 16 q / 8 kv heads, D=128, bf16,
    4096 + 3 prompt tokens, k=4; checked on every 61st query and the last 9
    (the raw tail and the block boundary before it)."""
    dt, B, Hkv, G, D, S = "bf16", 1, 8, 2, 128, 4096 + 3
    ks, vs, (kx, vx) = streams(dt, B, Hkv, S, D, 4, 77, oracle)
    ks.append(kx)
    vs.append(vx)
    g = torch.Generator(device=DEV).manual_seed(78)
    q = (torch.randn((B, Hkv * G, S, D), generator=g, device=DEV) / math.sqrt(D)).to(
        torch.bfloat16)
    out = codec_prefill_attention(q, ks, vs)
    rows = list(range(0, S, 61)) + list(range(S - 9, S))
    ref = causal_reference(to_values(q), view_oracle(oracle, ks), view_oracle(oracle, vs), 0,
                           D ** -0.5, rows=rows)
    check(to_values(out)[:, :, rows], ref, dt)


def test_prefill_distance_from_the_reference_prefill(oracle):
    """How far the default prefill (causal attention on the archive's stored
    rows) sits from the reference's prefill (SDPA on the read() view, the
    reconstruction rounded to bf16) at the C5 prompt's geometry: both within
    the contract of the exact (fp64) reconstruction's attention, and from
    each other within the sum of their distances to it.  Prints the three
    distances (relative to max|out|)."""
    dt, B, Hkv, G, D, S = "bf16", 1, 8, 2, 128, 1024 + 3
    ks, vs, (kx, vx) = streams(dt, B, Hkv, S, D, 4, 91, oracle)
    ks.append(kx)
    vs.append(vx)
    g = torch.Generator(device=DEV).manual_seed(92)
    q = (torch.randn((B, Hkv * G, S, D), generator=g, device=DEV) / math.sqrt(D)).to(
        torch.bfloat16)
    arch = codec_prefill_attention(q, ks, vs)
    kview, vview = ks.read(), vs.read()
    ref_view = torch.nn.functional.scaled_dot_product_attention(
        q, kview.repeat_interleave(G, dim=1), vview.repeat_interleave(G, dim=1), is_causal=True)
    ks.discard_view()
    vs.discard_view()
    rows = list(range(0, S, 17)) + list(range(S - 9, S))
    exact = causal_reference(to_values(q), view_oracle(oracle, ks), view_oracle(oracle, vs), 0,
                             D ** -0.5, rows=rows)
    a, v = to_values(arch)[:, :, rows], to_values(ref_view)[:, :, rows]
    m = np.abs(exact).max()
    d_arch, d_view = np.abs(a - exact).max() / m, np.abs(v - exact).max() / m
    d_between = np.abs(a - v).max() / m
    print(f"prefill distances / max|out|: archive-exact {d_arch:.2e}, view-exact {d_view:.2e}, "
          f"archive-view {d_between:.2e}", flush=True)
    check(to_values(arch)[:, :, rows], exact, dt)
    assert d_view <= 4e-3
    assert d_between <= d_arch + d_view + 1e-6


def tiny_qwen3(dtype=torch.bfloat16, attn=None):
    from transformers import Qwen3Config, Qwen3ForCausalLM
    torch.manual_seed(3)
    cfg = Qwen3Config(vocab_size=256, hidden_size=256, intermediate_size=512,
                      num_hidden_layers=2, num_attention_heads=8, num_key_value_heads=4,
                      head_dim=64, max_position_embeddings=1024, tie_word_embeddings=True)
    if attn is not None:
        cfg._attn_implementation = attn
    m = Qwen3ForCausalLM(cfg).eval()
    m.generation_config.eos_token_id = None
    return m.to(DEV, dtype)


def test_patched_prefill_runs_on_the_archive():
    """With the attention patch, a batched prefill on int8 jpeg layers
    attends on the archive (no view, counted per module) and its logits and
    the next decode steps track the model's own attention on the view."""
    pytest.importorskip("transformers")
    from flashcodec_amd import patch_attention as pa
    g = torch.Generator().manual_seed(9)
    ids = torch.randint(1, 256, (3, 8 * 21 + 5), generator=g).to(DEV)
    forced = torch.randint(1, 256, (3, 3), generator=g).to(DEV)
    cfg = dict(mode="jpeg", block_size=8, keep_freqs=4, quant_bits=8)
    model = tiny_qwen3()
    fc.apply_flash_codec(model, materialization_free=True, **cfg)
    results = {}
    for on_archive in (False, True):
        prev = pa.set_prefill_on_archive(on_archive)
        try:
            with torch.no_grad():
                out = model(input_ids=ids, use_cache=True)
                logits = [out.logits[:, -1].float()]
                pkv = out.past_key_values
                for layer in pkv.layers:
                    assert layer._key_stream._rec is None and layer.keys is None
                for i in range(3):
                    out = model(input_ids=forced[:, i:i + 1], past_key_values=pkv,
                                use_cache=True)
                    logits.append(out.logits[:, -1].float())
        finally:
            pa.set_prefill_on_archive(prev)
        results[on_archive] = (logits, out.logits[:, -1].float())
    counts = [getattr(m, "_flashcodec_prefills", 0) for m in fc.find_attention_modules(model)]
    assert counts == [1, 1]
    for a, b in zip(results[False][0], results[True][0]):
        assert (a - b).abs().max().item() <= 3e-2 * a.abs().max().item()
    fc.remove_flash_codec(model)


CFG_I8 = dict(mode="jpeg", block_size=8, keep_freqs=4, quant_bits=8)


def _prefill_logits(model, ids, mask=None, on_archive=True):
    from flashcodec_amd import patch_attention as pa
    prev = pa.set_prefill_on_archive(on_archive)
    try:
        with torch.no_grad():
            out = model(input_ids=ids, attention_mask=mask, use_cache=True)
    finally:
        pa.set_prefill_on_archive(prev)
    return out.logits.float()


def test_prefill_switch_off_is_the_reference_prefill():
    """set_prefill_on_archive(False): the patched prefill is the reference's
    own (the model's attention on the reconstructed view), so its logits equal
    those of the codec cache without the attention patch, bit for bit."""
    pytest.importorskip("transformers")
    ids = torch.randint(1, 256, (2, 8 * 13 + 3), generator=torch.Generator().manual_seed(4)).to(DEV)
    ref_model, model = tiny_qwen3(), tiny_qwen3()
    fc.apply_flash_codec(ref_model, **CFG_I8)
    fc.apply_flash_codec(model, materialization_free=True, **CFG_I8)
    with torch.no_grad():
        ref = ref_model(input_ids=ids, use_cache=True).logits.float()
    got = _prefill_logits(model, ids, on_archive=False)
    assert torch.equal(ref, got)
    assert [getattr(m, "_flashcodec_prefills", 0) for m in fc.find_attention_modules(model)] \
        == [0, 0]


def test_padded_prompt_prefill_keeps_its_mask():
    """A batch-1 prompt with padded (masked) key columns: the archive prefill
    applies only the plain causal mask, so the patch runs the model's own
    attention with the mask; the logits equal those with the archive prefill
    switched off, and no module counts an archive prefill."""
    pytest.importorskip("transformers")
    ids = torch.randint(1, 256, (1, 8 * 9 + 5), generator=torch.Generator().manual_seed(6)).to(DEV)
    mask = torch.ones_like(ids)
    mask[:, :3] = 0                               # left padding
    model = tiny_qwen3()
    fc.apply_flash_codec(model, materialization_free=True, **CFG_I8)
    off = _prefill_logits(model, ids, mask, on_archive=False)
    on = _prefill_logits(model, ids, mask, on_archive=True)
    assert torch.equal(on, off)
    assert [getattr(m, "_flashcodec_prefills", 0) for m in fc.find_attention_modules(model)] \
        == [0, 0]


def test_explicit_causal_mask_prefill_on_the_archive():
    """Eager-attention models pass the plain causal mask explicitly (an
    additive float mask) even when nothing is padded: the patch recognises it
    and runs the prefill on the archive (batch 2), whose logits track the
    model's own attention on the view; a padded batch keeps the masked
    path."""
    pytest.importorskip("transformers")
    ids = torch.randint(1, 256, (2, 8 * 11 + 6), generator=torch.Generator().manual_seed(8)).to(DEV)
    model = tiny_qwen3(attn="eager")
    fc.apply_flash_codec(model, materialization_free=True, **CFG_I8)
    off = _prefill_logits(model, ids, on_archive=False)
    on = _prefill_logits(model, ids, on_archive=True)
    counts = [getattr(m, "_flashcodec_prefills", 0) for m in fc.find_attention_modules(model)]
    assert counts == [1, 1]
    assert (on - off).abs().max().item() <= 3e-2 * off.abs().max().item()
    mask = torch.ones_like(ids)
    mask[1, :4] = 0
    assert torch.equal(_prefill_logits(model, ids, mask, on_archive=True),
                       _prefill_logits(model, ids, mask, on_archive=False))
    counts = [getattr(m, "_flashcodec_prefills", 0) for m in fc.find_attention_modules(model)]
    assert counts == [1, 1]
