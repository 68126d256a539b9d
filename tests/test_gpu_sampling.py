"""The device sampler (mcamd_sample_tokens) against the oracle (oracle/sampling.py): identical
token ids wherever the oracle's best score leads the runner-up by more than float32 rounding can
move it; exact argmax at temperature 0; per-row independence; counters advancing on the device;
and the empirical distribution of many draws against softmax(logits / T)."""
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
