"""Generation primitives over the KV path: next-token sampling and the cached ``Decoder``
(modelcore/generate.py:18-94).

``Decoder`` prefills a prompt at batch 1, replicates its cache into ``num_samples`` rows with the
HIP replication kernel (``KVCache.prefill``), then steps every row one position per call. Several
prompts are prefilled together as one packed sequence (``PackedPrefill``: no padding), each
written straight into its first sample row and copied into the others
(``KVCache.fill_sample_rows``), the rows right-ragged; row ``p * num_samples + s`` is sample ``s``
of prompt ``p``.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from modelcore_amd.cache import PackedPrefill


@torch.inference_mode()
def sample_next_token(logits, rng, temperature=1.0, top_k=None):
    """(B, vocab) logits -> (B, 1) token ids: argmax at temperature 0, else a multinomial draw
    from softmax(logits / temperature), over the top_k logits when top_k is set."""
    assert temperature >= 0.0, "temperature must be non-negative"
    if temperature == 0.0:
        return torch.argmax(logits, dim=-1, keepdim=True)
    if top_k is not None and top_k > 0:
        vals, idx = torch.topk(logits, min(top_k, logits.size(-1)), dim=-1)
        choice = torch.multinomial(F.softmax(vals / temperature, dim=-1), num_samples=1,
                                   generator=rng)
        return idx.gather(1, choice)
    return torch.multinomial(F.softmax(logits / temperature, dim=-1), num_samples=1,
                             generator=rng)


class Decoder:
    """Batch-1 prefill, replication into num_samples rows, then one position per step()."""

    @torch.inference_mode()
    def __init__(self, model, manager, tokens, *, num_samples=1, max_tokens=None, device=None):
        self.model = model
        device = device or model.get_device()
        if isinstance(tokens[0], int):
            prefill = manager.new_kv_cache(model, batch_size=1, seq_len=len(tokens), device=device)
            ids = torch.tensor([tokens], dtype=torch.long, device=device)
            logits = model.last_logits(ids, prefill, torch.tensor([len(tokens) - 1]))
            self._logits = logits.expand(num_samples, -1)
            length = len(tokens) + max_tokens if max_tokens is not None \
                else model.config.sequence_len
            self.kv_cache = manager.new_kv_cache(model, batch_size=num_samples, seq_len=length,
                                                 device=device)
            self.kv_cache.prefill(prefill)
            return
        # Several prompts: one packed forward of all their tokens (no padding) that writes prompt
        # p's K/V straight into row p * num_samples of the decode cache (PackedPrefill, the varlen
        # operator), then copies of that row into the prompt's other sample rows -- in place of
        # the reference's per-prompt batch-1 prefill and prefill_row copies
        # (modelcore/generate.py:67-80), with no transient cache and no host reads.
        prompts = [list(p) for p in tokens]
        lengths = [len(p) for p in prompts]
        assert min(lengths) > 0, "empty prompt"
        longest = max(lengths)
        length = longest + max_tokens if max_tokens is not None else model.config.sequence_len
        self.kv_cache = manager.new_kv_cache(model, batch_size=len(prompts) * num_samples,
                                             seq_len=length, device=device)
        packed = PackedPrefill(self.kv_cache, [p * num_samples for p in range(len(prompts))],
                               lengths)
        ids = torch.tensor([t for prompt in prompts for t in prompt], dtype=torch.long,
                           device=device).unsqueeze(0)
        logits = model.last_logits(ids, packed, None)
        self.kv_cache.fill_sample_rows(lengths, num_samples)
        self._logits = logits.repeat_interleave(num_samples, dim=0)

    @property
    def logits(self):
        """Next-token logits (rows, vocab), refreshed by step()."""
        return self._logits

    @torch.inference_mode()
    def step(self, token_column):
        """One next-token id per row (list or (rows,) tensor); advances every row one position."""
        device = self.model.get_device()
        if torch.is_tensor(token_column):
            ids = token_column.to(device=device, dtype=torch.long).view(-1, 1)
        else:
            ids = torch.tensor(token_column, dtype=torch.long, device=device).unsqueeze(1)
        self._logits = self.model.forward(ids, kv_cache=self.kv_cache)[:, -1, :]
        return self._logits

    def capture(self, sampler, temperature=1.0, top_k=None):
        """A ``CapturedStep`` of this decoder: each call samples from the current logits on the
        device (over the top_k largest logits of each row when top_k is set, as
        ``sample_next_token``) and steps every row, as one graph replay."""
        return CapturedStep(self, sampler, temperature, top_k)


class CapturedStep:
    """One whole decode step -- model forward on every row's last token, device sampling of the
    next token, cache advance -- recorded once as a HIP graph and replayed per position.

    The reference's step (modelcore/generate.py:82-94) returns to the host between positions: it
    builds the token column from a Python list and samples with torch.multinomial. Here the
    tokens stay on the device: the sampled column is written into the buffer the next replay
    reads, so a replay is one graph launch with no host sync. What the graph cannot do -- move the
    cache's host-side position and check it against the rotary table and the cache length -- runs
    on the host around each replay, without touching the device.

    Needs a uniform cache (every row at one position, as after ``KVCache.prefill``): a ragged
    cache checks its rotary positions with a device read, which a graph cannot hold. Every
    attention layer must take the fused pre-attention step, which reads its RoPE positions from
    ``cache_seqlens`` on the device (the separate ops would keep the capture's position). The first
    column is drawn from the decoder's current logits when the step is built, and building runs
    one real step (the warm-up that settles lazily created buffers) before the capture.
    """

    @torch.inference_mode()
    def __init__(self, decoder, sampler, temperature=1.0, top_k=None):
        self.decoder, self.sampler, self.temperature = decoder, sampler, float(temperature)
        self.top_k = top_k
        cache = decoder.kv_cache
        if cache.uniform_pos() is None:
            raise ValueError("CapturedStep needs a uniform cache (rows at one position)")
        model = decoder.model
        # The separate RoPE ops slice the tables at the host position of the capture, which a
        # replay would reuse at every later position; the fused step reads positions on the device.
        unfused = [b.layer_idx for b in model.body.blocks if not b.mixer.fuses_epilogue(cache)]
        if unfused:
            raise ValueError(f"CapturedStep needs every attention layer on the fused pre-attention "
                             f"step (RoPE at positions read on the device); layers {unfused} run "
                             f"the separate ops, whose RoPE would stay at the capture's position")
        self._rotary_len = min(b.mixer.rope.cos.size(1) for b in model.body.blocks)
        self.tokens = sampler(decoder.logits, self.temperature, self.top_k).view(-1, 1).clone()
        side = torch.cuda.Stream(device=self.tokens.device)
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            self._check()
            self._body()  # warm-up: a real step
        torch.cuda.current_stream().wait_stream(side)
        self.graph = torch.cuda.CUDAGraph()
        pos = cache._pos_uniform
        self._check()
        with torch.cuda.graph(self.graph, stream=side):
            self._body()
        cache._pos_uniform = pos  # the capture ran no kernel: the cache did not move
        torch.cuda.current_stream().wait_stream(side)

    def _check(self):
        cache = self.decoder.kv_cache
        pos = cache.uniform_pos()
        assert pos + 1 <= self._rotary_len, \
            f"Sequence length grew beyond the rotary embeddings cache: {pos + 1} > {self._rotary_len}"
        assert pos + 1 <= cache.max_seq_len, \
            f"Sequence length {pos + 1} exceeds cache length {cache.max_seq_len}"

    def _body(self):
        logits = self.decoder.model.forward(self.tokens, kv_cache=self.decoder.kv_cache)[:, -1, :]
        self.decoder._logits = logits
        self.tokens.copy_(self.sampler(logits, self.temperature, self.top_k).view(-1, 1))

    def __call__(self):
        """Feed the current token column, sample the next into ``self.tokens`` (returned; it is
        overwritten by the next call), advance every row one position."""
        self._check()
        self.graph.replay()
        self.decoder.kv_cache._pos_uniform += 1
        return self.tokens
