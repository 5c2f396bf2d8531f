"""GPU: the per-32 absmax int8 jpeg archive (quant_group=32: one fp32 scale
per 32 features of every (block, frequency) row, the quantizer flashcodec
README.md:487-494 describes and does not ship) against the oracle.

Archive codes and scales, the reconstructed view and the standalone
quantize_coeffs(group=32) are bit-exact against oracle.jpeg_encode_grouped /
grouped_coefficients (the pinned row quantizer applied per group); decode
attention, fused steps and graph replays on these archives are checked in
test_gpu_attention / test_gpu_configs / test_gpu_graph under their "i8g"
ids.  Here also: a patched model generates on grouped layers through the
codec-domain attention and tracks the materialised path.
"""

import numpy as np
import pytest
import torch

import flashcodec_amd as fc
from flashcodec_amd.cache import _CodecStream
from tests.conftest import to_values, torch_dtype

pytestmark = pytest.mark.gpu
DEV = "cuda"


def bits(a):
    a = np.ascontiguousarray(a, np.float32)
    return a.view(np.uint32)


def _values(oracle, shape, dt, seed):
    """AR(1) tokens with per-feature gains spread over 1e-3..1e2, so the
    32-feature groups of a row have very different absmax."""
    rng = np.random.default_rng(seed)
    gain = np.exp(rng.uniform(-7, 4.6, shape[:-2] + (1, shape[-1]))).astype(np.float32)
    return oracle.round_to(oracle.ar1(shape, 0.9, seed) * gain, dt)


CASES = [
    # dt, r, k, (B, H, S, D), feed (None: one append)
    ("bf16", 8, 4, (2, 4, 8 * 40 + 5, 128), None),
    ("f16", 8, 2, (1, 2, 8 * 25 + 3, 64), 7),
    ("f32", 8, 4, (2, 2, 8 * 16, 256), None),
    ("bf16", 16, 3, (1, 3, 16 * 12 + 9, 96), 5),
    ("f16", 4, 4, (2, 1, 4 * 30 + 1, 32), 1),
    ("f32", 24, 5, (1, 2, 24 * 6 + 4, 64), None),   # streaming encode (r > 16)
]


@pytest.mark.parametrize("case", CASES, ids=[f"{c[0]}-r{c[1]}k{c[2]}-D{c[3][3]}-f{c[4]}"
                                             for c in CASES])
def test_grouped_archive_and_read_match_oracle(case, oracle):
    dt, r, k, shape, feed = case
    print(f"case grouped archive {case}", flush=True)
    xv = _values(oracle, shape, dt, 3 + r + k)
    x = torch.from_numpy(xv).to(torch_dtype(dt)).to(DEV)
    st = _CodecStream(fc.make_codec("jpeg", block_size=r, keep_freqs=k, quant_bits=8,
                                    quant_group=32))
    if feed is None:
        st.append(x)
    else:
        for t in range(0, shape[2], feed):
            st.append(x[:, :, t:t + feed])
    n = shape[2] // r
    assert st.n_blocks == n and st._scales.shape[-1] == shape[3] // 32
    basis = fc.dct_basis(r, k).numpy()
    coef, codes, scales = oracle.jpeg_encode_grouped(xv[:, :, :n * r], r, k, basis, dt)
    assert np.array_equal(st._coeffs[:, :, :n].cpu().numpy(), codes)
    assert np.array_equal(bits(st._scales[:, :, :n].cpu().numpy()), bits(scales))
    rec = oracle.jpeg_decode(oracle.grouped_coefficients(codes, scales), r, basis, dt)
    got = to_values(st.read())
    assert np.array_equal(bits(got[:, :, :n * r]), bits(rec))
    assert np.array_equal(bits(got[:, :, n * r:]), bits(xv[:, :, n * r:]))
    # the grouped archive is never coarser than one scale per row
    _, row_codes, row_scales = oracle.jpeg_encode(xv[:, :, :n * r], r, k, basis, dt, quant=True)
    err_g = np.abs(oracle.grouped_coefficients(codes, scales) - coef)
    err_r = np.abs(row_codes * row_scales[..., None] - coef)
    if shape[3] > 32:
        assert err_g.mean() < err_r.mean()
    else:                                         # one group per row: the row quantizer
        assert np.array_equal(codes, row_codes)


@pytest.mark.parametrize("dt", ["f32", "f16", "bf16"])
def test_quantize_coeffs_group_matches_oracle(dt, oracle):
    """quantize_coeffs / dequantize_coeffs with group=32 on coefficient
    tensors: per-32 codes and scales of the pinned quantizer, and the
    dequantised values are the dtype products per group."""
    rng = np.random.default_rng(5)
    cv = oracle.round_to(rng.standard_normal((3, 7, 4, 160)).astype(np.float32)
                         * np.exp(rng.uniform(-5, 5, (1, 1, 1, 160))).astype(np.float32), dt)
    c = torch.from_numpy(cv).to(torch_dtype(dt)).to(DEV)
    q, s = fc.quantize_coeffs(c, 8, group=32)
    assert s.shape == (3, 7, 4, 5)
    codes, scales = oracle.quantize(cv.reshape(3, 7, 4, 5, 32), dt)
    assert np.array_equal(q.cpu().numpy(), codes.reshape(cv.shape))
    assert np.array_equal(bits(s.cpu().numpy()), bits(scales))
    deq = fc.dequantize_coeffs(q, s, torch.float32).cpu().numpy()
    assert np.array_equal(bits(deq), bits(oracle.grouped_coefficients(q.cpu().numpy(), scales)))
    with pytest.raises(ValueError):
        fc.quantize_coeffs(c[..., :100], 8, group=32)


def test_grouped_codec_validation():
    with pytest.raises(AssertionError):
        fc.make_codec("jpeg", quant_group=32)                 # needs quant_bits=8
    with pytest.raises(ValueError):
        fc.make_codec("png", quant_group=32)
    st = _CodecStream(fc.make_codec("jpeg", keep_freqs=2, quant_bits=8, quant_group=32))
    with pytest.raises(ValueError, match="multiple"):
        st.append(torch.randn(1, 1, 16, 40, device=DEV))
    c = fc.make_codec("jpeg", keep_freqs=2, quant_bits=8, quant_group=32)
    assert "quant_group=32" in repr(c)


def test_grouped_generation_tracks_materialised_path():
    """A tiny Qwen3 (bf16, batch 3) generating on grouped int8 layers: the
    codec-domain attention (prefill on the view, decode steps on the archive)
    tracks the materialised codec path while the greedy tokens agree."""
    pytest.importorskip("transformers")
    from tests.test_gpu_hf import VOCAB, tiny_qwen3
    ids = torch.randint(1, VOCAB, (3, 45), generator=torch.Generator().manual_seed(2)).to(DEV)
    cfg = dict(mode="jpeg", block_size=8, keep_freqs=4, quant_bits=8, quant_group=32)
    runs = {}
    for mf in (False, True):
        model = tiny_qwen3()
        fc.apply_flash_codec(model, materialization_free=mf, **cfg)
        with torch.no_grad():
            runs[mf] = model.generate(input_ids=ids, do_sample=False, max_new_tokens=12,
                                      output_logits=True, return_dict_in_generate=True,
                                      pad_token_id=0)
        if mf:
            steps = [getattr(m, "_flashcodec_codec_steps", 0)
                     for m in fc.find_attention_modules(model)]
            assert all(s == 11 for s in steps), steps
            cache = model._flashcodec["caches"][-1]
            assert cache.layers[0].codec.quant_group == 32
    n_same = 0
    for a, b in zip(runs[False].logits, runs[True].logits):
        err = (a.float() - b.float()).abs().max().item()
        assert err <= 3e-2 * a.float().abs().max().item(), (n_same, err)
        if not torch.equal(a.argmax(-1), b.argmax(-1)):
            break
        n_same += 1
    assert n_same >= 4
