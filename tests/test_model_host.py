"""The model harness around the KV path, on the CPU with the oracle operator plugged in
(``attention=oracle.sdpa_fallback.flash_attn``): this pins the harness's own arithmetic (embedding,
RoPE, QK-norm, x1.2, KV sharing, output gate, MLP, softcap, cache bookkeeping) before the GPU
tests run the same model on the HIP operator.

* The reference's goldens (tests/golden/README.md): no-cache logits within 2e-6 of what the
  reference produced (the reference asserts bit-identity on the machine that wrote them; here 85%
  of the logits differ in the last one to four bits, the signature of a different CPU matmul
  kernel, while a planted mistake moves them by 0.2 or more); a prefill followed by cached
  single-token steps reproduces them to 1e-4.
* Decoder at temperature 0 equals a naive no-cache greedy loop (modelcore/tests/test_generate.py:
  49-67), on "awake" weights (zero-init projections given small random values, as at
  test_generate.py:187-201), so attention actually affects the tokens.
* Multi-prompt (right-ragged) decode equals each prompt decoded alone (test_generate.py:220-234).
"""
import pytest
import torch

import _goldens
from modelcore_amd.generate import sample_next_token
from modelcore_amd.model import ComponentSpec, ModelConfig, ModelManager, kv_cache_spec
from modelcore_amd.runtime import Runtime
from oracle import sdpa_fallback

CPU = torch.device("cpu")


@pytest.fixture(autouse=True)
def cpu_cache_copies(monkeypatch):
    """KVCache's row copies run the HIP replication kernel; on CPU caches the oracle's restated
    copy stands in for it, so Decoder can be exercised here."""
    from modelcore_amd.cache import KVCache
    monkeypatch.setattr(KVCache, "_replicate_from",
                        lambda self, other, r0, n, t, src_row=0:
                        sdpa_fallback.replicate_rows(self, other, r0, n, t, src_row))


def manager():
    return ModelManager(Runtime(torch.float32), attention=sdpa_fallback.flash_attn)


GOLDEN_ATOL = 2e-6


@pytest.mark.parametrize("name", _goldens.GOLDENS)
def test_no_cache_logits_equal_the_reference_goldens(name):
    model, idx, logits = _goldens.build(name, manager(), CPU)
    with torch.no_grad():
        torch.testing.assert_close(model(idx), logits, atol=GOLDEN_ATOL, rtol=0)


@pytest.mark.parametrize("plant", ["rope_sign", "no_qk_scale", "window_plus_one", "gqa_roll"])
def test_planted_harness_mistakes_miss_the_golden(plant, monkeypatch):
    """Each plausible slip in the harness moves the golden logits far beyond the tolerance."""
    import modelcore_amd.model as M
    name = "v2_llama_kvshare_win_gated_block.pt"
    if plant == "rope_sign":
        rot = M.rotate
        monkeypatch.setattr(M, "rotate", lambda x, c, s: rot(x, c, -s))
    model, idx, logits = _goldens.build(name, manager(), CPU)
    for blk in model.body.blocks:
        if plant == "window_plus_one":
            blk.mixer.window += 1
        if plant == "no_qk_scale":
            blk.mixer.norm = M.RMSNorm(None)
            blk.mixer.norm.forward = lambda x: M.F.rms_norm(x, (x.size(-1),)) / 1.2
        if plant == "gqa_roll" and blk.mixer.produces_kv:
            w = blk.mixer.c_k.weight
            w.data = w.data.view(2, 16, -1).flip(0).reshape_as(w)
    with torch.no_grad():
        assert (model(idx) - logits).abs().max() > 1e-2


@pytest.mark.parametrize("name", _goldens.GOLDENS)
def test_prefill_then_cached_steps_reproduce_the_golden_logits(name):
    """A 4-token prefill into the cache, then one cached step per remaining token."""
    mgr = manager()
    model, idx, logits = _goldens.build(name, mgr, CPU)
    B, T = idx.shape
    cache = mgr.new_kv_cache(model, batch_size=B, seq_len=T)
    with torch.no_grad():
        parts = [model(idx[:, :4], kv_cache=cache)]
        for t in range(4, T):
            parts.append(model(idx[:, t:t + 1], kv_cache=cache))
    assert cache.get_pos() == T
    torch.testing.assert_close(torch.cat(parts, dim=1), logits, atol=1e-4, rtol=0)


def tiny_config(window=8, kv_share=False, gate=False, n_layer=4):
    blocks = []
    for i in range(n_layer):
        consumer = kv_share and i % 2 == 1
        mixer = ComponentSpec("attention", {
            "n_head": 4, "n_kv_head": 2, "head_dim": 16, "window": window if i % 4 != 3 else -1,
            "kv_slot": (i - 1) // 2 if consumer else (i // 2 if kv_share else None),
            "produces_kv": not consumer,
            "features": [ComponentSpec("output_gate", {"granularity": "head", "block_size": None,
                                                       "in_channels": None})] if gate else []})
        blocks.append(ComponentSpec("block", {"layer_idx": i, "features": [], "mixer": mixer,
                                              "ffn": ComponentSpec("gated_mlp", {
                                                  "activation": "silu", "hidden_dim": 96})}))
    return ModelConfig(sequence_len=64, vocab_size=100, n_embd=48,
                       shared={"rope": ComponentSpec("rotary", {"head_dim": 16, "over_compute": 10}),
                               "norm": ComponentSpec("rms_norm", {"eps": None})},
                       input=ComponentSpec("token_embedding", {"smear": False}),
                       body=ComponentSpec("stack", {"blocks": blocks, "features": []}),
                       output=ComponentSpec("lm_head", {"softcap": 15}))


def awake(model, seed=0):
    """Give every all-zero parameter small random values (test_generate.py:187-201)."""
    g = torch.Generator().manual_seed(seed + 1)
    with torch.no_grad():
        for p in model.parameters():
            if p.numel() and p.abs().sum() == 0:
                p.copy_((torch.randn(p.shape, generator=g) * 0.1).to(p.dtype))
    return model


def naive_greedy(model, tokens, n):
    ids = torch.tensor([tokens], dtype=torch.long)
    out = []
    with torch.no_grad():
        for _ in range(n):
            nxt = sample_next_token(model(ids)[:, -1, :], rng=None, temperature=0.0)
            ids = torch.cat((ids, nxt), dim=1)
            out.append(nxt.item())
    return out


def cached_greedy(mgr, model, tokens, n):
    dec = mgr.new_decoder(model, tokens, num_samples=1, max_tokens=n)
    out = []
    for _ in range(n):
        tok = sample_next_token(dec.logits, rng=None, temperature=0.0).item()
        out.append(tok)
        dec.step([tok])
    return out


@pytest.mark.parametrize("kv_share,gate", [(False, False), (True, False), (True, True)])
def test_decoder_matches_naive_greedy_on_awake_weights(kv_share, gate):
    mgr = manager()
    model = awake(mgr.create_model(tiny_config(kv_share=kv_share, gate=gate), device=CPU, seed=0))
    prompt = [5, 17, 3, 99, 42, 8, 61, 2, 13, 77]
    assert cached_greedy(mgr, model, prompt, 12) == naive_greedy(model, prompt, 12)


def test_multi_prompt_decode_matches_each_prompt_alone():
    mgr = manager()
    model = awake(mgr.create_model(tiny_config(kv_share=True), device=CPU, seed=0))
    prompts = [[1, 2], [3, 4, 5, 6, 7], [8, 9, 10, 11, 12, 13, 14, 15, 16],
               [2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13]]
    dec = mgr.new_decoder(model, prompts, num_samples=2, max_tokens=10)
    assert dec.kv_cache.uniform_pos() is None
    rows = [[] for _ in range(len(prompts) * 2)]
    for _ in range(10):
        nxt = sample_next_token(dec.logits, rng=None, temperature=0.0)
        for r, t in enumerate(nxt.view(-1).tolist()):
            rows[r].append(t)
        dec.step(nxt.view(-1))
    for p, prompt in enumerate(prompts):
        alone = cached_greedy(mgr, model, prompt, 10)
        assert rows[2 * p] == alone and rows[2 * p + 1] == alone, f"prompt {p}"


def test_kv_cache_spec_counts_distinct_slots():
    mgr = manager()
    model = mgr.create_model(tiny_config(kv_share=True, n_layer=6), device=CPU, seed=0)
    assert [s.kv_slot for s in model.layer_specs()] == [0, 0, 1, 1, 2, 2]
    assert kv_cache_spec(model.layer_specs()) == {"n_kv_head": 2, "head_dim": 16,
                                                  "num_kv_slots": 3}
    cache = mgr.new_kv_cache(model, batch_size=3, seq_len=20)
    assert cache.k_cache.shape == (3, 3, 20, 2, 16) and cache.k_cache.dtype == torch.float32


def test_seed_zero_init_follows_the_reference_scheme():
    """Init distributions of modelcore/components/*.py: wte N(0, 0.8), q/k/v U(+-sqrt(3/n_embd)),
    c_proj and down_proj zero, lm_head N(0, 0.001); same seed, same weights."""
    mgr = manager()
    a = mgr.create_model(tiny_config(), device=CPU, seed=0)
    b = mgr.create_model(tiny_config(), device=CPU, seed=0)
    for (ka, va), (kb, vb) in zip(a.state_dict().items(), b.state_dict().items()):
        assert ka == kb and torch.equal(va, vb)
    blk = a.body.blocks[0]
    bound = 3 ** 0.5 * 48 ** -0.5
    assert blk.mixer.c_q.weight.abs().max() <= bound and blk.mixer.c_q.weight.std() > bound / 3
    assert not blk.mixer.c_proj.weight.any() and not blk.ffn.down_proj.weight.any()
    assert abs(float(a.embedding.wte.weight.detach().std()) - 0.8) < 0.05
    assert abs(float(a.unembedding.lm_head.weight.detach().std()) - 0.001) < 2e-4


def test_the_default_operator_refuses_cpu_tensors():
    """Without an injected operator the model runs the HIP kernels only: CPU tensors raise."""
    mgr = ModelManager(Runtime(torch.float32))
    model = mgr.create_model(tiny_config(), device=CPU, seed=0)
    with pytest.raises(RuntimeError, match="ROCm device"):
        model(torch.tensor([[1, 2, 3]]))


def test_batched_prompt_prefill_equals_one_prefill_per_prompt():
    """The Decoder's batched prefill (one packed forward writing each prompt's K/V in place,
    then copies into the other sample rows) leaves the caches and first logits the reference's
    per-prompt prefill + prefill_row leave
    (modelcore/generate.py:67-80), within fp32 rounding; rows end at their own lengths."""
    mgr = manager()
    model = awake(mgr.create_model(tiny_config(kv_share=True), device=CPU, seed=0))
    prompts = [[4, 8, 15], [16, 23, 42, 4, 8, 15, 16], [1]]
    S, extra = 2, 5
    dec = mgr.new_decoder(model, prompts, num_samples=S, max_tokens=extra)
    assert dec.kv_cache.cache_seqlens.tolist() == [3, 3, 7, 7, 1, 1]
    assert dec.kv_cache.uniform_pos() is None
    ref = mgr.new_kv_cache(model, batch_size=len(prompts) * S, seq_len=7 + extra)
    ref_logits = []
    for p, prompt in enumerate(prompts):
        one = mgr.new_kv_cache(model, batch_size=1, seq_len=len(prompt))
        with torch.no_grad():
            ref_logits.append(model(torch.tensor([prompt]), kv_cache=one)[:, -1])
        for s in range(S):
            ref.prefill_row(p * S + s, one)
    assert ref.cache_seqlens.tolist() == dec.kv_cache.cache_seqlens.tolist()
    for r in range(len(prompts) * S):
        n = int(ref.cache_seqlens[r])
        torch.testing.assert_close(dec.kv_cache.k_cache[:, r, :n], ref.k_cache[:, r, :n],
                                   rtol=1e-5, atol=1e-6)
        torch.testing.assert_close(dec.kv_cache.v_cache[:, r, :n], ref.v_cache[:, r, :n],
                                   rtol=1e-5, atol=1e-6)
    want = torch.cat(ref_logits).repeat_interleave(S, 0)
    torch.testing.assert_close(dec.logits, want, rtol=1e-5, atol=1e-6)


def test_prefill_rows_refuses_what_it_cannot_place():
    mgr = manager()
    model = mgr.create_model(tiny_config(), device=CPU, seed=0)
    src = mgr.new_kv_cache(model, batch_size=2, seq_len=6)
    with pytest.raises(AssertionError, match="prompts x"):
        mgr.new_kv_cache(model, batch_size=3, seq_len=8).prefill_rows(src, [3, 6], 2)
    with pytest.raises(AssertionError, match="exceeds cache length"):
        mgr.new_kv_cache(model, batch_size=2, seq_len=4).prefill_rows(src, [3, 6], 1)
    dst = mgr.new_kv_cache(model, batch_size=2, seq_len=8)
    dst.advance(1)
    with pytest.raises(AssertionError, match="non-empty"):
        dst.prefill_rows(src, [3, 6], 1)


def test_packed_prefill_refuses_what_it_cannot_place():
    from modelcore_amd.cache import PackedPrefill
    mgr = manager()
    model = mgr.create_model(tiny_config(), device=CPU, seed=0)
    cache = mgr.new_kv_cache(model, batch_size=4, seq_len=8)
    with pytest.raises(AssertionError, match="distinct"):
        PackedPrefill(cache, [1, 1], [3, 4])
    with pytest.raises(AssertionError, match="out of range"):
        PackedPrefill(cache, [0, 4], [3, 4])
    with pytest.raises(AssertionError, match="empty prompt"):
        PackedPrefill(cache, [0, 1], [3, 0])
    with pytest.raises(AssertionError, match="exceeds cache length"):
        PackedPrefill(cache, [0, 1], [3, 9])
    cache.cache_seqlens[2] = 5
    cache._pos_uniform = None
    with pytest.raises(AssertionError, match="non-empty"):
        PackedPrefill(cache, [0, 2], [3, 4])
    PackedPrefill(cache, [0, 3], [3, 4])  # rows 0 and 3 are empty: accepted


def test_packed_prefill_moves_each_row_to_its_prompts_length():
    """A packed forward over prompts placed in rows 3 and 1 of a 4-row cache: those rows end at
    their prompts' lengths, the others stay empty (ragged host mirror); covering every row with
    equal lengths leaves the cache uniform. The last-token logits equal each prompt's own."""
    from modelcore_amd.cache import PackedPrefill
    mgr = manager()
    model = awake(mgr.create_model(tiny_config(kv_share=True), device=CPU, seed=0))
    cache = mgr.new_kv_cache(model, batch_size=4, seq_len=12)
    prompts = [[4, 8, 15, 16], [23, 42]]
    packed = PackedPrefill(cache, [3, 1], [4, 2])
    with torch.no_grad():
        logits = model.last_logits(torch.tensor([prompts[0] + prompts[1]]), packed, None)
    assert cache.cache_seqlens.tolist() == [0, 2, 0, 4] and cache.uniform_pos() is None
    for p, prompt in enumerate(prompts):
        one = mgr.new_kv_cache(model, batch_size=1, seq_len=len(prompt))
        with torch.no_grad():
            want = model(torch.tensor([prompt]), kv_cache=one)[:, -1]
        torch.testing.assert_close(logits[p:p + 1], want, rtol=1e-5, atol=1e-6)
        row = [3, 1][p]
        n = len(prompt)
        torch.testing.assert_close(cache.k_cache[:, row, :n], one.k_cache[:, 0, :n], rtol=1e-5,
                                   atol=1e-6)
    full = mgr.new_kv_cache(model, batch_size=2, seq_len=12)
    with torch.no_grad():
        model.last_logits(torch.tensor([[1, 2, 3, 4, 5, 6]]), PackedPrefill(full, [1, 0], [3, 3]),
                          None)
    assert full.uniform_pos() == 3 and full.cache_seqlens.tolist() == [3, 3]


def test_interleaved_gate_up_weights_split_back_into_gate_and_up():
    """interleave_gate_up puts 64 gate rows, then the 64 up rows of the same units, block after
    block; split_gate_up recovers gate and up of a product with it exactly (CPU)."""
    from modelcore_amd.kernels.linear import interleave_gate_up, split_gate_up
    g = torch.Generator().manual_seed(1)
    wg, wu = torch.randn(192, 32, generator=g), torch.randn(192, 32, generator=g)
    w = interleave_gate_up(wg, wu)
    assert torch.equal(w[:64], wg[:64]) and torch.equal(w[64:128], wu[:64])
    assert torch.equal(w[320:], wu[128:])
    x = torch.randn(3, 5, 32, generator=g)
    gate, up = split_gate_up(x @ w.T)
    torch.testing.assert_close(gate.reshape(3, 5, 192), x @ wg.T, atol=1e-5, rtol=0)
    torch.testing.assert_close(up.reshape(3, 5, 192), x @ wu.T, atol=1e-5, rtol=0)
    with pytest.raises(ValueError):
        interleave_gate_up(wg[:100], wu[:100])


def test_tiled_weights_round_trip_and_hold_64x128_blocks():
    """tile_weight stores (n, k) as (n/64, k/128, 64, 128) blocks, block [g][s] being rows
    64g.., columns 128s..; untile_weight restores the row-major weight exactly (CPU)."""
    from modelcore_amd.kernels.linear import tile_weight, untile_weight
    w = torch.arange(192 * 384, dtype=torch.float32).reshape(192, 384)
    t = tile_weight(w)
    assert t.shape == (3, 3, 64, 128) and t.is_contiguous()
    assert torch.equal(t[1, 2], w[64:128, 256:384])
    assert torch.equal(untile_weight(t), w)
    with pytest.raises(ValueError):
        tile_weight(w[:100])


def test_stepping_past_the_cache_raises_before_any_write():
    """The reference fails at the cache write past T_max (modelcore/cache.py:105 for a prefill
    row, an index error in the operator's append); the harness checks the room first, from the
    host mirror, so the kernels never see such a step."""
    mgr = manager()
    model = mgr.create_model(tiny_config(), device=CPU, seed=0)
    dec = mgr.new_decoder(model, [5, 17, 3], num_samples=2, max_tokens=2)
    dec.step([1, 2])
    dec.step([3, 4])
    before = dec.kv_cache.k_cache.clone()
    with pytest.raises(AssertionError, match="exceeds cache length"):
        dec.step([5, 6])
    assert torch.equal(dec.kv_cache.k_cache, before) and dec.kv_cache.get_pos() == 5
    ragged = mgr.new_decoder(model, [[5, 17, 3], [9]], num_samples=1, max_tokens=1)
    ragged.step([1, 2])
    with pytest.raises(AssertionError, match="exceeds cache length"):
        ragged.step([3, 4])


def test_captured_step_refuses_layers_on_the_separate_rope_ops():
    """A captured step replays whatever the capture recorded: the separate RoPE ops slice the
    tables at the host position of that moment, so only layers on the fused step (positions
    read on the device) may be captured."""
    mgr = manager()  # the oracle operator: no fused pre-attention step
    model = mgr.create_model(tiny_config(), device=CPU, seed=0)
    dec = mgr.new_decoder(model, [5, 17, 3], num_samples=2, max_tokens=4)
    with pytest.raises(ValueError, match="fused pre-attention"):
        dec.capture(lambda logits, t: logits.argmax(-1))
    for blk in model.body.blocks:
        blk.mixer.epilogue = object()
    model.set_fused_epilogue(False)
    with pytest.raises(ValueError, match=r"layers \[0, 1, 2, 3\]"):
        dec.capture(lambda logits, t: logits.argmax(-1))


def test_linear_workspace_keeps_outgrown_buffers_alive(monkeypatch):
    """A graph captured with the skinny GEMM's split-K workspace holds its address: when a larger
    call replaces the buffer, the old one must stay allocated (not return to the allocator)."""
    from modelcore_amd.kernels import linear as lin
    monkeypatch.setattr(lin, "_WS", {})
    monkeypatch.setattr(lin, "_RETIRED", [])
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: False)
    dev = torch.device("cpu", 0)
    small = lin._workspace(dev, 1000)
    assert lin._workspace(dev, 500) is small
    big = lin._workspace(dev, small.numel() + 1)
    assert big is not small and big.numel() >= 2 * small.numel()
    assert any(t is small for t in lin._RETIRED)


def test_checked_mode_raises_on_positions_past_the_cache(monkeypatch):
    """Opt-in checked mode of the operator: positions read back on the host, IndexError before
    any launch, as the reference's append raises (modelcore/kernels/flash_attn.py:336-346)."""
    from modelcore_amd.kernels import flash_attn as fa
    seen = []
    monkeypatch.setattr(fa._ext, "require_rocm", lambda *a, **k: None)
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: False)
    monkeypatch.setattr(fa._ext, "lib", lambda: seen.append("launch") or (_ for _ in ()).throw(
        RuntimeError("no launch expected")))
    fa.set_checked(True)
    try:
        q = torch.zeros(2, 1, 4, 16)
        kc = torch.zeros(2, 8, 2, 16)
        k = torch.zeros(2, 1, 2, 16)
        with pytest.raises(IndexError, match="outside the cache of 8"):
            fa.flash_attn_with_kvcache(q, kc, kc.clone(), k=k, v=k.clone(),
                                       cache_seqlens=torch.tensor([3, 8], dtype=torch.int32))
        with pytest.raises(IndexError):
            fa.flash_attn_with_kvcache(q.expand(2, 2, 4, 16), kc, kc.clone(),
                                       k=k.expand(2, 2, 2, 16), v=k.expand(2, 2, 2, 16),
                                       cache_seqlens=torch.tensor([0, 7], dtype=torch.int32))
        assert not seen
    finally:
        fa.set_checked(False)
