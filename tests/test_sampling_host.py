"""The sampling oracle (oracle/sampling.py) on the CPU: Philox4x32-10 against the known-answer
vectors published with the Random123 library (Salmon et al., SC 2011), and the Gumbel-max draw
against the softmax distribution it must follow."""
import numpy as np
import pytest
import torch

from oracle import sampling as S

KATS = [
    ((0, 0, 0, 0), (0, 0), (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
    ((0xFFFFFFFF,) * 4, (0xFFFFFFFF,) * 2, (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
    ((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344), (0xA4093822, 0x299F31D0),
     (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1)),
]


@pytest.mark.parametrize("ctr,key,want", KATS)
def test_philox_known_answers(ctr, key, want):
    got = S.philox4x32_10(np.array([ctr], dtype=np.uint64), np.array([key], dtype=np.uint64))[0]
    assert [int(x) for x in got] == list(want)


def test_uniforms_are_open_interval_float32_values():
    u = S.uniforms(seed=123, offset=7, vocab=4099)
    assert u.shape == (4099,) and (u > 0).all() and (u < 1).all()
    assert np.array_equal(u, u.astype(np.float32).astype(np.float64))
    assert abs(u.mean() - 0.5) < 0.02


def test_gumbel_max_draws_follow_softmax():
    logits = np.array([[0.3, -1.0, 2.0, 0.0, 1.1, -0.4, 0.9, -2.0]])
    for temperature in (1.0, 0.5):
        p = np.exp(logits[0] / temperature)
        p /= p.sum()
        n = 20000
        counts = np.zeros(8)
        for off in range(n):
            ids, _ = S.sample(logits, [99], [off], temperature)
            counts[ids[0]] += 1
        assert np.max(np.abs(counts / n - p)) < 0.015, (counts / n, p)


def test_temperature_zero_is_the_first_argmax():
    logits = np.array([[1.0, 3.0, 3.0, -1.0], [0.0, 0.0, 0.0, 0.0]])
    ids, _ = S.sample(logits, [1, 2], [0, 0], 0.0)
    assert ids.tolist() == [1, 0]


def test_rows_depend_only_on_their_own_seed_and_offset():
    g = np.random.default_rng(0)
    logits = g.standard_normal((6, 50))
    seeds, offs = [11, 12, 13, 14, 15, 16], [0, 3, 3, 9, 0, 1]
    ids, _ = S.sample(logits, seeds, offs, 1.0)
    for b in range(6):
        alone, _ = S.sample(logits[b:b + 1], [seeds[b]], [offs[b]], 1.0)
        assert alone[0] == ids[b]


def test_the_device_sampler_refuses_cpu_tensors():
    from modelcore_amd.sampling import PhiloxSampler
    with pytest.raises(RuntimeError, match="ROCm device"):
        PhiloxSampler(2, torch.device("cpu"))
