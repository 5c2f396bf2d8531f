"""GPU: the device-side structural operations (fc_gather_segments) under
the cache's batch gathers, capacity growth and crops: byte-exact against
torch's index_select / slicing, in place and out of place, with repeated
and permuted indices, odd segment sizes, and replayed from a HIP graph."""

import pytest
import torch

import flashcodec_amd as fc
from flashcodec_amd import _native as N
from flashcodec_amd.cache import FlashCodecLayer, _CodecStream, _gather

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _filled(shape, dtype, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    if dtype == torch.int8:
        return torch.randint(-127, 128, shape, generator=g, device=DEV, dtype=torch.int8)
    return torch.randn(shape, generator=g, device=DEV).to(dtype)


@pytest.mark.parametrize("dtype,tail", [(torch.int8, (4, 128)), (torch.float32, (3, 1)),
                                        (torch.float16, (5,)), (torch.bfloat16, (7, 24)),
                                        (torch.int8, (3, 5))])
@pytest.mark.parametrize("idx", [[2, 0, 3, 1], [1, 1, 3, 0], [0, 1, 2, 3], [3, 3, 3, 3]])
def test_in_place_gather_matches_index_select(dtype, tail, idx):
    """In place (a same-size reorder): every listed row index order, with
    repeats, over (B, H, cap, ...) buffers whose live prefix is n rows; rows
    past the prefix are untouched."""
    B, H, cap, n = 4, 3, 16, 11
    t = _filled((B, H, cap) + tail, dtype, 1)
    before = t.clone()
    ix = torch.tensor(idx, device=DEV)
    _gather(t, t, ix, n)
    assert torch.equal(t[:, :, :n], before[:, :, :n].index_select(0, ix))
    assert torch.equal(t[:, :, n:], before[:, :, n:])


@pytest.mark.parametrize("B_out,idx", [(6, [0, 0, 1, 1, 2, 2]), (2, [3, 1]), (4, None)])
def test_out_of_place_gather_and_prefix_copy(B_out, idx):
    """Out of place: batch expansion and selection, and the identity prefix
    copy of a capacity growth into a larger buffer."""
    B, H, D = 4, 2, 40
    src = _filled((B, H, 16, 3, D), torch.float16, 2)
    dst = torch.zeros((B_out, H, 32, 3, D), dtype=torch.float16, device=DEV)
    ix = None if idx is None else torch.tensor(idx, device=DEV)
    _gather(dst, src, ix, 13)
    ref = src[:, :, :13] if ix is None else src[:, :, :13].index_select(0, ix)
    assert torch.equal(dst[:, :, :13], ref)
    assert not dst[:, :, 13:].any()


def test_out_of_range_indices_are_skipped():
    """The kernel never reads outside its source: a row index outside
    [0, B) leaves that destination row as it was (the Python layer rejects
    such indices before calling)."""
    B, H = 3, 2
    t = _filled((B, H, 8, 32), torch.float32, 3)
    before = t.clone()
    ix = torch.tensor([2, -1, 7], device=DEV)
    es = t.element_size()
    N.check(N.lib().fc_gather_segments(t.data_ptr(), t.stride(0) * es, t.stride(1) * es,
                                       t.data_ptr(), t.stride(0) * es, t.stride(1) * es,
                                       ix.data_ptr(), B, B, H, 8 * 32 * es,
                                       N.stream_ptr(t.device)), "gather")
    assert torch.equal(t[0], before[2])
    assert torch.equal(t[1:], before[1:])
    st = _CodecStream(fc.make_codec("jpeg", block_size=8, keep_freqs=2))
    st.append(torch.randn(B, H, 20, 32, device=DEV))
    with pytest.raises(IndexError):
        st.select_batch(torch.tensor([0, 3, 1]))


@pytest.mark.parametrize("cfg", [dict(mode="jpeg", block_size=8, keep_freqs=4, quant_bits=8),
                                 dict(mode="png", block_size=8, keep_ratio=0.5)])
def test_beam_reorder_replays_from_a_graph(cfg):
    """A same-size beam reorder of a codec layer (archives and tail
    gathered in place, no allocation) captured once as a HIP graph and
    replayed with new indices in its index tensor: every replay equals the
    eager index_select of the previous state, with eager work between."""
    torch.manual_seed(4)
    B, H, S, D = 4, 2, 8 * 9 + 5, 64
    layer = FlashCodecLayer(**cfg)
    k, v = torch.randn(B, H, S, D, device=DEV), torch.randn(B, H, S, D, device=DEV)
    layer.update(k, v)
    for st in (layer._key_stream, layer._value_stream):
        st.discard_view()
    layer.keys = layer.values = None
    idx = torch.zeros(B, dtype=torch.int64, device=DEV)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        layer._pair.select_batch(idx)
    torch.cuda.synchronize()

    def state():
        out = []
        for st in (layer._key_stream, layer._value_stream):
            out += [t[:, :, :st.n_blocks].clone() for t in st._archive_tensors()]
            out.append(st.raw.clone())
        return out

    g = torch.Generator().manual_seed(5)
    for _ in range(4):
        before = state()
        perm = torch.randint(0, B, (B,), generator=g)
        idx.copy_(perm.to(DEV))
        graph.replay()
        torch.cuda.synchronize()
        pd = perm.to(DEV)
        for a, b in zip(state(), before):
            assert torch.equal(a, b.index_select(0, pd))
        _ = (torch.randn(64, 64, device=DEV) @ torch.randn(64, 64, device=DEV)).sum()
        torch.cuda.synchronize()
    assert layer._key_stream.seq_len == S


def test_crop_reconstructs_the_boundary_into_the_tail():
    """A crop inside the archive: the kept tokens of the boundary block come
    back as the raw tail, equal to the reconstructed view's tokens, with no
    reconstruction buffer built."""
    torch.manual_seed(6)
    cfg = dict(mode="jpeg", block_size=8, keep_freqs=3, quant_bits=8)
    x = torch.randn(2, 3, 8 * 7 + 2, 32, device=DEV, dtype=torch.bfloat16)
    ref = _CodecStream(fc.make_codec(**cfg))
    ref.append(x)
    view = ref.read().clone()
    st = _CodecStream(fc.make_codec(**cfg))
    st.append(x)
    st.crop(-(8 * 3 + 5))                       # 58 - 29: keep 8*3 + 5 tokens
    assert st._rec is None and st.n_blocks == 3 and st.seq_len == 8 * 3 + 5
    assert torch.equal(st.raw, view[:, :, 8 * 3:8 * 3 + 5])
    assert torch.equal(st.read(), view[:, :, :8 * 3 + 5])
