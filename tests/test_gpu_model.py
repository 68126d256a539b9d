"""The model harness on the GPU, attention through the HIP kernels, against the same model on the
CPU with the oracle operator (tests/test_model_host.py pins that one) and against the reference's
goldens.

* Goldens (fp32, head_dim 16): no-cache logits, and a prefill plus cached single-token steps,
  match the reference's logits to 1e-4.
* The README quickstart model (12 layers, 768 wide, 12/12 heads of 64, gated SiLU MLP 2048, vocab
  32768, softcap 15, fp32, seed-0 weights drawn on the CPU): batch 2, prompts of 16 tokens, 64
  greedy tokens -- the token ids equal the CPU oracle's exactly, with the seed-0 weights (whose
  zero-init projections make attention irrelevant) and with awake weights (where it is not).
* A mixed-window, KV-sharing stack in bf16 (head_dim 128, GQA 12/4): logits of a prefill and of
  cached decode steps stay within bf16 tolerance of the fp32 CPU oracle.
"""
import pytest
import torch

import _goldens
from modelcore_amd.generate import sample_next_token
from modelcore_amd.model import ComponentSpec, ModelConfig, ModelManager
from modelcore_amd.runtime import Runtime
from oracle import sdpa_fallback
from test_model_host import awake

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda", 0)
CPU = torch.device("cpu")


def _note(*a):
    print("case:", *a, flush=True)


def gpu_manager(dtype=torch.float32):
    return ModelManager(Runtime(dtype))


def cpu_manager():
    return ModelManager(Runtime(torch.float32), attention=sdpa_fallback.flash_attn)


@pytest.fixture
def cpu_cache_copies(monkeypatch):
    from modelcore_amd.cache import KVCache
    real = KVCache._replicate_from

    def copy(self, other, r0, n, t, src_row=0):
        if self.k_cache.device.type == "cpu":
            return sdpa_fallback.replicate_rows(self, other, r0, n, t, src_row)
        return real(self, other, r0, n, t, src_row)

    monkeypatch.setattr(KVCache, "_replicate_from", copy)


@pytest.mark.parametrize("name", _goldens.GOLDENS)
def test_goldens_no_cache_and_cached_on_the_gpu(name):
    _note("golden", name)
    mgr = gpu_manager()
    model, idx, logits = _goldens.build(name, mgr, DEV)
    idx = idx.to(DEV)
    with torch.no_grad():
        full = model(idx).cpu()
        torch.testing.assert_close(full, logits, atol=1e-4, rtol=0)
        cache = mgr.new_kv_cache(model, batch_size=idx.size(0), seq_len=idx.size(1))
        parts = [model(idx[:, :5], kv_cache=cache)]
        for t in range(5, idx.size(1)):
            parts.append(model(idx[:, t:t + 1], kv_cache=cache))
    torch.testing.assert_close(torch.cat(parts, dim=1).cpu(), logits, atol=1e-4, rtol=0)


def quickstart_config():
    hd = 64
    blocks = [ComponentSpec("block", {
        "layer_idx": i, "features": [],
        "mixer": ComponentSpec("attention", {"n_head": 12, "n_kv_head": 12, "head_dim": hd,
                                             "window": -1, "kv_slot": None, "produces_kv": True,
                                             "features": []}),
        "ffn": ComponentSpec("gated_mlp", {"activation": "silu", "hidden_dim": 2048})})
        for i in range(12)]
    return ModelConfig(sequence_len=1024, vocab_size=32768, n_embd=768, pad_vocab_size_to=64,
                       shared={"rope": ComponentSpec("rotary", {"head_dim": hd, "over_compute": 10}),
                               "norm": ComponentSpec("rms_norm", {"eps": None})},
                       input=ComponentSpec("token_embedding", {"smear": False}),
                       body=ComponentSpec("stack", {"blocks": blocks, "features": []}),
                       output=ComponentSpec("lm_head", {"softcap": 15}))


def greedy_ids(mgr, model, prompts, n):
    dec = mgr.new_decoder(model, prompts, num_samples=1, max_tokens=n)
    rows = [[] for _ in prompts]
    for _ in range(n):
        nxt = sample_next_token(dec.logits, rng=None, temperature=0.0)
        for r, t in enumerate(nxt.view(-1).tolist()):
            rows[r].append(t)
        dec.step(nxt.view(-1))
    return rows


@pytest.mark.parametrize("wake", [False, True], ids=["seed0", "awake"])
def test_quickstart_greedy_ids_equal_the_cpu_oracle(wake, cpu_cache_copies):
    _note("quickstart greedy", "awake" if wake else "seed0")
    cfg = quickstart_config()
    cpu_mgr = cpu_manager()
    cpu_model = cpu_mgr.create_model(cfg, device=CPU, seed=0)
    if wake:
        awake(cpu_model)
    gpu_mgr = gpu_manager()
    gpu_model = gpu_mgr.create_model(cfg, device=DEV, seed=0)
    gpu_model.load_state_dict(cpu_model.state_dict())
    g = torch.Generator().manual_seed(0)
    prompts = torch.randint(0, cfg.vocab_size, (2, 16), generator=g).tolist()
    want = greedy_ids(cpu_mgr, cpu_model, prompts, 64)
    got = greedy_ids(gpu_mgr, gpu_model, prompts, 64)
    assert got == want


def mixed_window_config(n_layer=8):
    """Layer i is global iff i % 4 == 3, else window 64; odd layers read the previous layer's
    slot."""
    blocks = []
    for i in range(n_layer):
        consumer = i % 2 == 1
        blocks.append(ComponentSpec("block", {
            "layer_idx": i, "features": [],
            "mixer": ComponentSpec("attention", {
                "n_head": 12, "n_kv_head": 4, "head_dim": 128,
                "window": -1 if i % 4 == 3 else 64, "kv_slot": (i - 1) // 2 if consumer else i // 2,
                "produces_kv": not consumer, "features": []}),
            "ffn": ComponentSpec("gated_mlp", {"activation": "silu", "hidden_dim": 768})}))
    return ModelConfig(sequence_len=512, vocab_size=512, n_embd=384,
                       shared={"rope": ComponentSpec("rotary", {"head_dim": 128,
                                                                "over_compute": 10}),
                               "norm": ComponentSpec("rms_norm", {"eps": None})},
                       input=ComponentSpec("token_embedding", {"smear": False}),
                       body=ComponentSpec("stack", {"blocks": blocks, "features": []}),
                       output=ComponentSpec("lm_head", {"softcap": 15}))


def test_mixed_window_kv_sharing_stack_in_bf16(cpu_cache_copies):
    _note("mixed-window bf16 stack")
    cfg = mixed_window_config()
    cpu_mgr = cpu_manager()
    cpu_model = awake(cpu_mgr.create_model(cfg, device=CPU, seed=0))
    gpu_mgr = gpu_manager(torch.bfloat16)
    gpu_model = gpu_mgr.create_model(cfg, device=DEV, seed=0)
    gpu_model.load_state_dict(cpu_model.state_dict())
    g = torch.Generator().manual_seed(1)
    B, P, steps = 4, 200, 6
    prompt = torch.randint(0, cfg.vocab_size, (B, P + steps), generator=g)
    cpu_cache = cpu_mgr.new_kv_cache(cpu_model, batch_size=B, seq_len=P + steps)
    gpu_cache = gpu_mgr.new_kv_cache(gpu_model, batch_size=B, seq_len=P + steps)
    assert gpu_cache.n_slots == 4 and gpu_cache.k_cache.dtype == torch.bfloat16
    with torch.no_grad():
        want = [cpu_model(prompt[:, :P], kv_cache=cpu_cache)[:, -1]]
        got = [gpu_model(prompt[:, :P].to(DEV), kv_cache=gpu_cache)[:, -1].cpu()]
        for t in range(P, P + steps):
            want.append(cpu_model(prompt[:, t:t + 1], kv_cache=cpu_cache)[:, -1])
            got.append(gpu_model(prompt[:, t:t + 1].to(DEV), kv_cache=gpu_cache)[:, -1].cpu())
    for i, (a, b) in enumerate(zip(got, want)):
        err = (a - b).abs().max().item()
        print(f"call {i}: logits max-abs {err:.4f} (scale {b.abs().max().item():.3f})", flush=True)
        # bf16 rounding of weights, activations and K/V against the fp32 CPU oracle: ~2e-3 on
        # logits of scale ~0.07
        assert err <= 5e-3, f"call {i}: logits max-abs {err}"
    assert gpu_cache.cache_seqlens.tolist() == [P + steps] * B


def test_sampling_decoder_rows_are_replicas_and_draws_are_reproducible():
    """The large-batch sampling flow at small scale (bf16, GQA 12/4, head_dim 128): one prompt
    prefilled at batch 1 and replicated to 8 rows gives 8 bit-identical caches and identical
    first logits; device sampling with per-row seeds then decodes the same tokens on a rerun, and
    rows that happen to draw the same tokens keep identical logits."""
    from modelcore_amd.sampling import PhiloxSampler
    _note("sampling decoder")
    cfg = mixed_window_config(n_layer=4)
    mgr = gpu_manager(torch.bfloat16)
    model = mgr.create_model(cfg, device=DEV, seed=0)
    awake(model)
    model.cache_inference_weights()
    prompt = torch.randint(0, cfg.vocab_size, (150,), generator=torch.Generator().manual_seed(2))

    def run():
        dec = mgr.new_decoder(model, prompt.tolist(), num_samples=8, max_tokens=12)
        kc = dec.kv_cache.k_cache
        assert all(torch.equal(kc[:, r, :150], kc[:, 0, :150]) for r in range(8))
        assert torch.equal(dec.logits, dec.logits[:1].expand(8, -1))
        sampler = PhiloxSampler(8, DEV, base_seed=40)
        toks = []
        for _ in range(12):
            t = sampler(dec.logits, 1.0).view(-1)
            toks.append(t.cpu())
            dec.step(t)
        return torch.stack(toks, dim=1)

    a, b = run(), run()
    assert torch.equal(a, b)
    assert len({tuple(r.tolist()) for r in a}) > 1  # different seeds diverge


def test_sampling_decoder_with_the_shared_prefix_matches_its_own_rows():
    """The same flow decoded twice, teacher-forced on one token stream: once with the attention
    taking the replicated prompt's K/V from row 0 (KVCache.shared_prefix, set by prefill; 32 rows
    x 3 query heads per KV head put the prompt on the matrix cores) and once with each row reading
    its own copy. The prefill logits are identical; the decode logits agree within the bf16
    rounding of the reordered sums."""
    from modelcore_amd.sampling import PhiloxSampler
    _note("sampling decoder, shared prefix")
    cfg = mixed_window_config(n_layer=4)
    mgr = gpu_manager(torch.bfloat16)
    model = mgr.create_model(cfg, device=DEV, seed=0)
    awake(model)
    model.cache_inference_weights()
    prompt = torch.randint(0, cfg.vocab_size, (600,), generator=torch.Generator().manual_seed(3))
    rows, steps = 32, 8
    shared = mgr.new_decoder(model, prompt.tolist(), num_samples=rows, max_tokens=steps)
    own = mgr.new_decoder(model, prompt.tolist(), num_samples=rows, max_tokens=steps)
    assert shared.kv_cache.shared_prefix == 600
    own.kv_cache.shared_prefix = 0
    assert torch.equal(shared.logits, own.logits)
    sampler = PhiloxSampler(rows, DEV, base_seed=7)
    for i in range(steps):
        t = sampler(shared.logits, 1.0).view(-1)
        shared.step(t)
        own.step(t)
        err = (shared.logits.float() - own.logits.float()).abs().max().item()
        scale = own.logits.float().abs().max().item()
        print(f"step {i}: logits max-abs {err:.5f} (scale {scale:.3f})", flush=True)
        assert err <= 0.05, f"step {i}: logits max-abs {err}"


def test_cached_inference_weights_give_identical_logits():
    """The bf16 weight copies give the logits of the per-call casts bit for bit; stacking the
    QKV and gate/up copies into one product each changes only the GEMM's summation order."""
    cfg = mixed_window_config(n_layer=2)
    mgr = gpu_manager(torch.bfloat16)
    model = awake(mgr.create_model(cfg, device=DEV, seed=0))
    idx = torch.randint(0, cfg.vocab_size, (2, 40), generator=torch.Generator().manual_seed(3)).to(DEV)
    with torch.no_grad():
        a = model(idx)
        model.cache_inference_weights(fuse=False)
        b = model(idx)
        model.cache_inference_weights()
        assert model.body.blocks[0].mixer._qkv is not None
        c = model(idx)
        model.drop_inference_weights()
        d = model(idx)
    assert torch.equal(a, b) and torch.equal(a, d)
    err = (a.float() - c.float()).abs().max().item()
    print(f"stacked projections: logits max-abs {err:.4f}", flush=True)
    assert err <= 0.05


def test_skinny_gemm_projections_match_the_library_gemm(monkeypatch):
    """With use_skinny_gemm, a decode-sized forward (32 rows) runs its projections through
    mcamd_linear_bf16; the logits match the F.linear ones up to the GEMMs' summation order."""
    from modelcore_amd.kernels import linear as lin
    cfg = mixed_window_config(n_layer=2)
    mgr = gpu_manager(torch.bfloat16)
    model = awake(mgr.create_model(cfg, device=DEV, seed=0))
    idx = torch.randint(0, cfg.vocab_size, (2, 16), generator=torch.Generator().manual_seed(4)).to(DEV)
    calls, gated = [], []
    real, real_gated = lin.linear_bf16, lin.linear_bf16_gated
    monkeypatch.setattr(lin, "linear_bf16", lambda *a, **k: (calls.append(1), real(*a, **k))[1])
    monkeypatch.setattr(lin, "linear_bf16_gated",
                        lambda *a, **k: (gated.append(1), real_gated(*a, **k))[1])
    with torch.no_grad():
        model.cache_inference_weights()
        a = model(idx)
        assert not calls and not gated
        model.use_skinny_gemm(True)
        b = model(idx)
        model.use_skinny_gemm(False)
    assert len(calls) >= 3 * 2  # qkv, c_proj, down of both layers (+ lm_head)
    assert len(gated) == 2  # gate/up with the SiLU product, one per layer
    err = (a.float() - b.float()).abs().max().item()
    print(f"skinny GEMM projections: logits max-abs {err:.4f}", flush=True)
    assert err <= 0.05


def test_fused_pre_attention_step_matches_the_separate_ops():
    """The same bf16 mixed-window, KV-sharing stack with the fused RoPE + QK-norm + x1.2 + append
    launch (the default) and with the reference's separate ops, fed the same tokens (a prefill,
    then cached single-token steps): caches and logits agree within bf16 rounding."""
    _note("fused vs separate pre-attention step")
    cfg = mixed_window_config()
    mgr = gpu_manager(torch.bfloat16)
    model = awake(mgr.create_model(cfg, device=DEV, seed=0))
    g = torch.Generator().manual_seed(4)
    B, P, steps = 3, 120, 8
    tokens = torch.randint(0, cfg.vocab_size, (B, P + steps), generator=g).to(DEV)
    runs = []
    for fused in (True, False):
        model.set_fused_epilogue(fused)
        cache = mgr.new_kv_cache(model, batch_size=B, seq_len=P + steps)
        with torch.no_grad():
            logits = [model(tokens[:, :P], kv_cache=cache)[:, -1]]
            for t in range(P, P + steps):
                logits.append(model(tokens[:, t:t + 1], kv_cache=cache)[:, -1])
        runs.append((torch.stack(logits).float(), cache))
    model.set_fused_epilogue(True)
    (la, ca), (lb, cb) = runs
    err = (la - lb).abs().max().item()
    print(f"logits max-abs fused vs separate: {err:.4f} (scale {lb.abs().max().item():.3f})",
          flush=True)
    assert err <= 0.1
    assert torch.equal(ca.cache_seqlens, cb.cache_seqlens)
    for a, b in ((ca.k_cache, cb.k_cache), (ca.v_cache, cb.v_cache)):
        assert (a.float() - b.float()).abs().max() <= 0.1


def test_fused_residual_steps_match_the_separate_ops():
    """With set_fused_residual (and the skinny GEMM), each residual add + RMS-norm is one launch
    that also sums c_proj's / down_proj's K-split partials, and the norm is carried to the next
    block and the lm_head: a prefill (rows > 64: the separate ops) then cached single-token steps
    (the fused launches) give the logits of the separate ops within bf16 rounding."""
    _note("fused residual steps")
    cfg = mixed_window_config(n_layer=4)
    mgr = gpu_manager(torch.bfloat16)
    model = awake(mgr.create_model(cfg, device=DEV, seed=0))
    model.cache_inference_weights()
    model.use_skinny_gemm(True)
    g = torch.Generator().manual_seed(6)
    B, P, steps = 4, 60, 6
    tokens = torch.randint(0, cfg.vocab_size, (B, P + steps), generator=g).to(DEV)
    runs = []
    for fused in (True, False):
        model.set_fused_residual(fused)
        cache = mgr.new_kv_cache(model, batch_size=B, seq_len=P + steps)
        with torch.no_grad():
            logits = [model(tokens[:, :P], kv_cache=cache)[:, -1]]
            for t in range(P, P + steps):
                logits.append(model(tokens[:, t:t + 1], kv_cache=cache)[:, -1])
            last = model.last_logits(tokens[:, :P], mgr.new_kv_cache(model, batch_size=B,
                                                                     seq_len=P),
                                     torch.full((B,), P - 1))
        runs.append((torch.stack(logits).float(), last.float()))
    model.set_fused_residual(False)
    (la, lla), (lb, llb) = runs
    assert torch.equal(la[0], lb[0]) and torch.equal(lla, llb)  # prefill: the separate ops
    err = (la - lb).abs().max().item()
    print(f"logits max-abs fused residual vs separate: {err:.4f} (scale "
          f"{lb.abs().max().item():.3f})", flush=True)
    assert err <= 0.1


@pytest.mark.parametrize("fast,top_k", [(False, None), (True, None), (True, 50)],
                         ids=["library-gemm", "skinny-fused-residual", "skinny-top_k"])
def test_captured_decode_step_replays_the_eager_steps(fast, top_k):
    """A whole decode step (forward, device sampling, advance) captured once as a HIP graph and
    replayed: the same tokens, logits and cache as the same steps run eagerly, and the host-side
    position kept in step with the device; also with the skinny GEMM and fused residual steps,
    and with the draw restricted to the top_k logits."""
    from modelcore_amd.sampling import PhiloxSampler
    _note("captured decode step", fast, top_k)
    cfg = mixed_window_config(n_layer=4)
    mgr = gpu_manager(torch.bfloat16)
    model = awake(mgr.create_model(cfg, device=DEV, seed=0))
    model.cache_inference_weights()
    model.use_skinny_gemm(fast)
    model.set_fused_residual(fast)
    prompt = torch.randint(0, cfg.vocab_size, (90,), generator=torch.Generator().manual_seed(5))
    R, n = 6, 10

    eager = mgr.new_decoder(model, prompt.tolist(), num_samples=R, max_tokens=n + 2)
    sampler = PhiloxSampler(R, DEV, base_seed=7)
    toks, logits = [], []
    for _ in range(n + 1):
        t = sampler(eager.logits, 1.0, top_k).view(-1)
        toks.append(t.clone())
        eager.step(t)
        logits.append(eager.logits.float().clone())

    dec = mgr.new_decoder(model, prompt.tolist(), num_samples=R, max_tokens=n + 2)
    step = dec.capture(PhiloxSampler(R, DEV, base_seed=7), 1.0, top_k)
    assert torch.equal(step.tokens.view(-1), toks[1])  # the warm-up ran the first step
    assert dec.kv_cache.get_pos() == 90 + 1
    for i in range(1, n):
        out = step()
        assert dec.kv_cache.get_pos() == 90 + 1 + i
        assert torch.equal(out.view(-1), toks[i + 1]), i
        err = (dec.logits.float() - logits[i]).abs().max().item()
        assert err <= 1e-2, (i, err)
    torch.cuda.synchronize()
    assert dec.kv_cache.cache_seqlens.tolist() == [90 + n] * R
    assert torch.equal(dec.kv_cache.k_cache[:, :, :90 + n], eager.kv_cache.k_cache[:, :, :90 + n])


def test_batched_multi_prompt_prefill_matches_one_prefill_per_prompt():
    """Ragged prompts prefilled together (one packed forward writing each prompt's K/V in place,
    PackedPrefill and the varlen operator) against the reference's flow of one prefill and
    prefill_row per prompt, bf16 on the GPU: the same lengths, caches and logits within bf16
    rounding, also after decode steps fed the same tokens."""
    _note("batched multi-prompt prefill")
    cfg = mixed_window_config(n_layer=4)
    mgr = gpu_manager(torch.bfloat16)
    model = awake(mgr.create_model(cfg, device=DEV, seed=0))
    g = torch.Generator().manual_seed(6)
    lengths, S, steps = [37, 150, 5, 88], 2, 4
    prompts = [torch.randint(0, cfg.vocab_size, (n,), generator=g).tolist() for n in lengths]
    dec = mgr.new_decoder(model, prompts, num_samples=S, max_tokens=steps + 1)
    ref = mgr.new_kv_cache(model, batch_size=len(prompts) * S, seq_len=150 + steps + 1)
    ref_logits = []
    with torch.no_grad():
        for p, prompt in enumerate(prompts):
            one = mgr.new_kv_cache(model, batch_size=1, seq_len=len(prompt))
            ref_logits.append(model(torch.tensor([prompt], device=DEV), kv_cache=one)[:, -1])
            for s in range(S):
                ref.prefill_row(p * S + s, one)
    assert dec.kv_cache.cache_seqlens.tolist() == ref.cache_seqlens.tolist()
    for r, n in enumerate(ref.cache_seqlens.tolist()):
        for a, b in ((dec.kv_cache.k_cache, ref.k_cache), (dec.kv_cache.v_cache, ref.v_cache)):
            # the packed path's products have other shapes than each prompt's (the library may
            # sum in another order) and it runs RoPE / QK-norm / x1.2 as separate ops, the
            # per-prompt path fused: the layers' outputs agree to about one bf16 unit of their
            # scale, which the later layers' K/V inherit (measured: at most 0.047 at scale ~3)
            x, y = a[:, r, :n].float(), b[:, r, :n].float()
            err = (x - y).abs().max().item()
            assert err <= 2 ** -5 * y.abs().max().item(), (r, err)
    want = torch.cat(ref_logits).repeat_interleave(S, 0).float()
    err = (dec.logits.float() - want).abs().max().item()
    print(f"prefill logits max-abs {err:.2e}", flush=True)
    assert err <= 2e-3
    feed = torch.randint(0, cfg.vocab_size, (steps, len(prompts) * S), generator=g).to(DEV)
    with torch.no_grad():
        for t in range(steps):
            a = dec.step(feed[t]).float()
            b = model(feed[t].view(-1, 1), kv_cache=ref)[:, -1].float()
            err = (a - b).abs().max().item()
            print(f"step {t}: logits max-abs {err:.2e}", flush=True)
            assert err <= 2e-3, t
