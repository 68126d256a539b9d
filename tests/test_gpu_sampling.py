"""The device sampler (mcamd_sample_tokens) against the oracle (oracle/sampling.py): identical
token ids wherever the oracle's best score leads the runner-up by more than float32 rounding can
move it, also with top_k (logits held in registers up to 32768 per row, read from memory past
that; rows with ties at the k-th value); exact argmax at temperature 0; per-row independence;
counters advancing on the device; and the empirical distribution of many draws against
softmax(logits / T)."""
import numpy as np
import pytest
import torch

from modelcore_amd.sampling import PhiloxSampler
from oracle import sampling as S

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


def _note(*a):
    print("case:", *a, flush=True)


@pytest.mark.parametrize("temperature", [1.0, 0.7])
def test_device_draws_equal_the_oracle(temperature):
    _note("sampler vs oracle", temperature)
    g = torch.Generator().manual_seed(5)
    B, V = 64, 32768
    sampler = PhiloxSampler(B, DEV, base_seed=1000)
    compared = 0
    for step in range(3):
        logits = (torch.randn(B, V, generator=g) * 3).float()
        ids = sampler(logits.to(DEV), temperature).view(-1).cpu().numpy()
        want, margin = S.sample(logits.numpy(), [1000 + r for r in range(B)], [step] * B,
                                temperature)
        ok = margin > 1e-3
        compared += int(ok.sum())
        assert np.array_equal(ids[ok], want[ok]), f"step {step}"
    assert compared >= 0.95 * 3 * B
    assert sampler.offsets.cpu().tolist() == [3] * B


def test_temperature_zero_is_torch_argmax():
    g = torch.Generator().manual_seed(6)
    logits = torch.randn(32, 1000, generator=g)
    logits[3, 10] = logits[3, 500] = 50.0  # a tie: the lower index wins, as torch.argmax
    sampler = PhiloxSampler(32, DEV)
    ids = sampler(logits.to(DEV), 0.0).view(-1).cpu()
    assert torch.equal(ids, torch.argmax(logits, dim=-1)) and ids[3] == 10


def test_a_rows_draw_does_not_depend_on_the_batch():
    g = torch.Generator().manual_seed(7)
    logits = torch.randn(16, 4096, generator=g).to(DEV)
    seeds = [77 + 3 * r for r in range(16)]
    together = PhiloxSampler(16, DEV, seeds=seeds)
    got = [together(logits).view(-1).cpu() for _ in range(4)]
    for r in (0, 5, 15):
        alone = PhiloxSampler(1, DEV, seeds=[seeds[r]])
        for step in range(4):
            assert alone(logits[r:r + 1]).item() == got[step][r].item()


def test_draws_follow_softmax():
    _note("sampler distribution")
    V, B, calls = 16, 4096, 8
    logits = torch.linspace(-2.0, 1.5, V).repeat(B, 1).to(DEV)
    sampler = PhiloxSampler(B, DEV, base_seed=31)
    counts = torch.zeros(V)
    for _ in range(calls):
        counts += torch.bincount(sampler(logits, 1.0).view(-1).cpu(), minlength=V).float()
    p = torch.softmax(torch.linspace(-2.0, 1.5, V), dim=0)
    assert (counts / (B * calls) - p).abs().max() < 0.01


@pytest.mark.parametrize("top_k", [1, 40, 1000, 32767])
def test_top_k_draws_equal_the_oracle(top_k):
    _note("sampler top_k vs oracle", top_k)
    g = torch.Generator().manual_seed(8)
    B, V = 64, 32768
    sampler = PhiloxSampler(B, DEV, base_seed=500)
    compared = 0
    for step in range(2):
        logits = (torch.randn(B, V, generator=g) * 3).float()
        ids = sampler(logits.to(DEV), 0.9, top_k=top_k).view(-1).cpu().numpy()
        want, margin = S.sample(logits.numpy(), [500 + r for r in range(B)], [step] * B, 0.9,
                                top_k=top_k)
        ok = margin > 1e-3
        compared += int(ok.sum())
        assert np.array_equal(ids[ok], want[ok]), f"step {step}"
        kept = np.stack([S.top_k_mask(logits[r].numpy(), top_k) for r in range(B)])
        assert kept[np.arange(B), ids].all()  # never a dropped logit
    assert compared >= 0.9 * 2 * B


def test_top_k_with_ties_and_a_vocabulary_read_from_memory():
    """Quantised logits (many ties at the k-th value: the lowest indices are kept) at a vocabulary
    that fits in registers and at one that does not (50000 logits per row)."""
    g = torch.Generator().manual_seed(9)
    for V in (4096, 50000):
        _note("sampler top_k ties, vocab", V)
        B = 16
        logits = torch.randint(-6, 7, (B, V), generator=g).float()
        sampler = PhiloxSampler(B, DEV, base_seed=900)
        for k in (5, 300):
            ids = sampler(logits.to(DEV), 1.0, top_k=k).view(-1).cpu().numpy()
            off = int(sampler.offsets[0].item()) - 1
            want, margin = S.sample(logits.numpy(), [900 + r for r in range(B)], [off] * B, 1.0,
                                    top_k=k)
            ok = margin > 1e-3
            assert ok.sum() >= B // 2
            assert np.array_equal(ids[ok], want[ok]), (V, k)
            kept = np.stack([S.top_k_mask(logits[r].numpy(), k) for r in range(B)])
            assert kept[np.arange(B), ids].all()
