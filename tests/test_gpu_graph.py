"""GPU: decode steps replayed from a captured HIP graph (device-side stream
counters) against the same steps run eagerly through the host-driven codec
path, on a tiny Qwen3 decoder with int8 jpeg (matrix-core attention),
unquantised jpeg, per-32-scaled int8 jpeg and png archives (vector-ALU
attention)."""

import pytest
import torch

import flashcodec_amd as fc
from flashcodec_amd import graph

pytestmark = pytest.mark.gpu

transformers = pytest.importorskip("transformers")


def tiny_qwen3(dtype, codec):
    from transformers import Qwen3Config, Qwen3ForCausalLM
    cfg = Qwen3Config(vocab_size=512, hidden_size=256, intermediate_size=512,
                      num_hidden_layers=2, num_attention_heads=8, num_key_value_heads=2,
                      head_dim=64, max_position_embeddings=4096, tie_word_embeddings=True)
    torch.manual_seed(0)
    model = Qwen3ForCausalLM(cfg).to(device="cuda", dtype=dtype).eval()
    fc.apply_flash_codec(model, materialization_free=True, **codec)
    return model


def prefill(model, prompt):
    with torch.no_grad():
        out = model(input_ids=prompt, use_cache=True, logits_to_keep=1)
    return out.past_key_values


I8 = dict(mode="jpeg", block_size=8, keep_freqs=4, quant_bits=8)
FP = dict(mode="jpeg", block_size=8, keep_freqs=4)
PNG = dict(mode="png", block_size=8, keep_ratio=0.5)
I8G = dict(I8, quant_group=32)


@pytest.mark.parametrize("dtype,codec", [(torch.float16, I8), (torch.bfloat16, I8),
                                         (torch.bfloat16, FP), (torch.float16, PNG),
                                         (torch.bfloat16, I8G)],
                         ids=["i8-f16", "i8-bf16", "fp-bf16", "png-f16", "i8g-bf16"])
def test_graph_replays_match_eager_steps(dtype, codec):
    model = tiny_qwen3(dtype, codec)
    g = torch.Generator().manual_seed(5)
    B, P, steps = 2, 29, 21                      # 29 + 21 tokens cross three block boundaries
    prompt = torch.randint(1, 512, (B, P), generator=g).cuda()
    forced = torch.randint(1, 512, (B, steps), generator=g).cuda()
    print(f"case graph decode {dtype} {codec}", flush=True)

    # eager, host-driven codec steps
    cache_e = prefill(model, prompt)
    ref = []
    with torch.no_grad():
        for i in range(steps):
            pos = torch.full((B, 1), P + i, dtype=torch.long, device="cuda")
            out = model(input_ids=forced[:, i:i + 1], position_ids=pos, past_key_values=cache_e,
                        use_cache=True, logits_to_keep=1)
            ref.append(out.logits[:, -1].float())

    # graph replays (one eager warm-up step on the decoder's stream first)
    cache_g = prefill(model, prompt)
    dec = graph.GraphDecoder(model, cache_g, forced[:, 0:1], position=P, max_new_tokens=steps,
                             warmup=1)
    for i in range(1, steps):
        dec.ids.copy_(forced[:, i:i + 1])
        dec.step()
        got = dec.logits[:, -1].float()
        torch.cuda.synchronize()
        # eager work between replays
        _ = (torch.randn(64, 64, device="cuda") @ torch.randn(64, 64, device="cuda")).sum()
        torch.cuda.synchronize()
        err = (got - ref[i]).abs().max().item()
        assert err <= 2e-2 * ref[i].abs().max().item(), f"replay {i}: max err {err:.3e}"
    dec.close()                                  # device counters == host counters
    for le, lg in zip(cache_e.layers, cache_g.layers):
        for se, sg in ((le._key_stream, lg._key_stream), (le._value_stream, lg._value_stream)):
            assert (se.n_blocks, se._n_raw, se.seq_len) == (sg.n_blocks, sg._n_raw, sg.seq_len)
    # layer 0's K/V depend on the forced tokens only: its archive is bit-exact
    l0e, l0g = cache_e.layers[0], cache_g.layers[0]
    for se, sg in ((l0e._key_stream, l0g._key_stream), (l0e._value_stream, l0g._value_stream)):
        n = se.n_blocks
        for te, tg in zip(se._archive_tensors(), sg._archive_tensors()):
            assert torch.equal(te[:, :, :n], tg[:, :, :n])
        assert torch.equal(se.raw, sg.raw)
    # the cache keeps working eagerly after the graph is released
    with torch.no_grad():
        pos = torch.full((B, 1), P + steps, dtype=torch.long, device="cuda")
        model(input_ids=forced[:, :1], position_ids=pos, past_key_values=cache_g, use_cache=True,
              logits_to_keep=1)
    assert cache_g.layers[0]._key_stream.seq_len == P + steps + 1
