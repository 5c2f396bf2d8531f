"""Greedy decoding with each decode step replayed from a captured HIP graph.

A decode step of a transformers causal LM patched with
``apply_flash_codec(..., materialization_free=True)`` is ~1,500 small kernel
launches issued from Python (the model's own ops), so it runs at the host's
dispatch rate, not the GPU's.  Capturing one step as a HIP graph and
replaying it removes the dispatch.  The codec side must then enqueue the same
work at every step: with ``prepare(cache, extra_tokens)`` every codec layer
keeps its (n_blocks, n_tail) counters in device memory, where
``fc_decode_step`` reads and advances them, and its archives are sized for
the tokens to come.  The host copies of the counters are advanced after each
executed step (``advance_host``), so ``seq_len``, ``read()`` and the other
stream APIs stay valid; ``release(cache)`` returns the layers to host-driven
steps.

Every store kind works (int8 jpeg on the matrix-core decode attention,
unquantised jpeg and png on the vector-ALU one; both merge in the same
launch).  This is not part of the reference, which has no graph path
(flashcodec/patch_attention.py decodes eagerly).
"""

import torch

from .cache import FlashCodecLayer


def _codec_layers(cache):
    return [layer for layer in getattr(cache, "layers", []) if isinstance(layer, FlashCodecLayer)]


def prepare(cache, extra_tokens):
    """Put the counters of every codec layer of `cache` on the device and
    grow its archives for `extra_tokens` more tokens.  Every layer must be a
    codec layer (other cache layers grow by concatenation, which a replayed
    graph cannot do) holding at least one archived block (a prefill of
    >= block_size tokens)."""
    layers = list(getattr(cache, "layers", []))
    if not layers or len(_codec_layers(cache)) != len(layers):
        raise NotImplementedError("graph decoding needs a cache whose layers are all codec layers")
    for layer in _codec_layers(cache):
        ks, vs = layer._key_stream, layer._value_stream
        c = ks.codec
        if ks.n_blocks < 1 or ks.n_blocks != vs.n_blocks or ks._n_raw != vs._n_raw:
            raise ValueError("graph decoding needs a prefill of at least one block per layer")
        r = c.block_size
        need = ks.n_blocks + (ks._n_raw + extra_tokens) // r + 1
        like = ks._archive_tensors()[0]
        for st in (ks, vs):
            st.discard_view()
            st._grow(need, like)
            st._tail_buffer(like)           # (B, H, r, D) in the stream dtype
        # (n_blocks, n_tail, overflow, padding)
        state = torch.tensor([ks.n_blocks, ks._n_raw, 0, 0], dtype=torch.int64,
                             device=like.device)
        ks._dev_state = vs._dev_state = state
        layer.keys = layer.values = None


def advance_host(cache, steps=1):
    """Advance the host counters of every codec layer by `steps` executed
    decode steps (one token each)."""
    for layer in _codec_layers(cache):
        ks, vs = layer._key_stream, layer._value_stream
        r = ks.codec.block_size
        t = ks._n_raw + steps
        full = t // r
        for st in (ks, vs):
            st.n_blocks += full
            st.n_archived += full * r
            st._n_raw = t - full * r


def release(cache, check=True):
    """Return the codec layers to host-driven decode steps.  With `check`,
    the device counters must equal the host ones and no step may have run
    past the archive capacity that prepare() reserved (a block completed
    beyond it was not archived, so the outputs of the steps since are wrong):
    RuntimeError otherwise."""
    for layer in _codec_layers(cache):
        ks, vs = layer._key_stream, layer._value_stream
        state = getattr(ks, "_dev_state", None)
        if state is None:
            continue
        ks._dev_state = vs._dev_state = None
        if check:
            nb, nt, overflow = (int(v) for v in state[:3].cpu())
            if overflow:
                raise RuntimeError("graph decode steps ran past the archive capacity reserved "
                                   "by prepare(); blocks past it were not archived")
            if (nb, nt) != (ks.n_blocks, ks._n_raw):
                raise RuntimeError(f"device counters ({nb}, {nt}) differ from the host's "
                                   f"({ks.n_blocks}, {ks._n_raw})")


class GraphDecoder:
    """Greedy decoding of `model` (patched with materialization_free=True)
    on the prefilled FlashCodecCache `cache`, one captured HIP graph per
    step::

        out = model(input_ids=prompt, use_cache=True, logits_to_keep=1)
        cache, nxt = out.past_key_values, out.logits[:, -1].argmax(-1, keepdim=True)
        dec = GraphDecoder(model, cache, nxt, position=prompt.shape[1], max_new_tokens=256)
        tokens = dec.generate(256)          # (B, 256) greedy continuation
        dec.close()

    `warmup` eager steps (which generate tokens like the replays) run before
    the capture; capture and replays run on the decoder's own stream.
    """

    def __init__(self, model, cache, input_ids, position, max_new_tokens, warmup=2):
        self.model, self.cache = model, cache
        dev = input_ids.device
        B = input_ids.shape[0]
        # decode steps (eager warm-up ones included) the archives are sized for
        self.capacity = int(max_new_tokens) + int(warmup)
        self.steps = 0
        prepare(cache, self.capacity)
        self.ids = input_ids.reshape(B, 1).clone()
        self.pos = torch.full((B, 1), int(position), dtype=torch.long, device=dev)
        cfg = model.config.get_text_config(decoder=True) if hasattr(model.config,
                                                                    "get_text_config") else model.config
        self.mask = {t: None for t in set(getattr(cfg, "layer_types", None) or ["full_attention"])}
        self.stream = torch.cuda.Stream(device=dev)
        self.pending = []       # tokens produced by the warm-up steps
        self.stream.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(self.stream):
            for _ in range(warmup):
                logits = self._forward()
                self._advance(logits)
        torch.cuda.current_stream(dev).wait_stream(self.stream)
        torch.cuda.synchronize(dev)
        self.graph = torch.cuda.CUDAGraph()
        with torch.no_grad(), torch.cuda.graph(self.graph, stream=self.stream):
            self.logits = self._forward()

    def _forward(self):
        with torch.no_grad():
            out = self.model(input_ids=self.ids, position_ids=self.pos, attention_mask=self.mask,
                             past_key_values=self.cache, use_cache=True, logits_to_keep=1)
        return out.logits

    def _advance(self, logits):
        self.steps += 1
        advance_host(self.cache)
        nxt = logits[:, -1].argmax(-1, keepdim=True)
        self.ids.copy_(nxt)
        self.pos.add_(1)
        self.pending.append(nxt.clone())

    def step(self):
        """Replay one decode step; returns the (B, 1) greedy tokens.  Raises
        RuntimeError once the steps reserved at construction (max_new_tokens
        + warmup) are used up: the archives hold no room for more blocks."""
        if self.steps >= self.capacity:
            raise RuntimeError(f"GraphDecoder reserved archive room for {self.capacity} decode "
                               "steps (max_new_tokens + warmup); build a new decoder to go on")
        with torch.cuda.stream(self.stream):
            self.graph.replay()
            self.steps += 1
            advance_host(self.cache)
            nxt = self.logits[:, -1].argmax(-1, keepdim=True)
            self.ids.copy_(nxt)
            self.pos.add_(1)
        torch.cuda.current_stream(self.ids.device).wait_stream(self.stream)
        return nxt

    def generate(self, n):
        """`n` greedy tokens (the warm-up steps' tokens first)."""
        toks = self.pending[:n]
        self.pending = self.pending[n:]
        while len(toks) < n:
            toks.append(self.step())
        return torch.cat(toks, dim=1)

    def close(self):
        """Release the graph and return the cache to host-driven steps."""
        torch.cuda.synchronize(self.ids.device)
        self.graph = None
        release(self.cache)
