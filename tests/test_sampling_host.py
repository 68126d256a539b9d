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


def test_top_k_mask_against_a_sort_with_ties():
    """The kept set is the k largest values, ties at the k-th value kept lowest index first --
    checked against a plain sort of (value, index) pairs on rows full of ties, and NaN kept last."""
    g = np.random.default_rng(1)
    for _ in range(200):
        V = int(g.integers(2, 40))
        row = g.integers(-3, 4, V).astype(np.float64)  # many equal values
        if g.random() < 0.2:
            row[g.integers(0, V)] = np.nan
        k = int(g.integers(1, V + 2))
        nan = np.isnan(row)
        pairs = sorted(range(V), key=lambda i: (np.inf if nan[i] else -row[i], bool(nan[i]), i))
        want = np.zeros(V, dtype=bool)
        want[pairs[:min(k, V)]] = True
        assert np.array_equal(S.top_k_mask(row, k), want), (row, k)
    assert S.top_k_mask(np.array([5.0, 3, 3, 3, 1]), 2).tolist() == [True, True, False, False, False]
    assert S.top_k_mask(np.array([np.nan, -np.inf, 0.0]), 2).tolist() == [False, True, True]
    assert S.top_k_mask(np.array([1.0, -0.0, 0.0]), 2).tolist() == [True, True, False]
    assert S.top_k_mask(np.array([1.0, 2.0]), None).all() and S.top_k_mask(np.array([1.0]), 0).all()


def test_top_k_draws_follow_softmax_over_the_kept_logits():
    """The reference's top_k branch (modelcore/generate.py:23-29) draws from softmax(top-k
    values / T): the restricted Gumbel-max must follow it, and never pick a dropped logit."""
    logits = np.array([[0.3, -1.0, 2.0, 0.0, 1.1, -0.4, 0.9, -2.0]])
    k = 3
    kept = np.argsort(-logits[0])[:k]
    p = np.zeros(8)
    p[kept] = np.exp(logits[0, kept] / 0.8)
    p /= p.sum()
    n = 20000
    counts = np.zeros(8)
    for off in range(n):
        ids, _ = S.sample(logits, [5], [off], 0.8, top_k=k)
        counts[ids[0]] += 1
    assert counts[np.setdiff1d(np.arange(8), kept)].sum() == 0
    assert np.max(np.abs(counts / n - p)) < 0.015, (counts / n, p)


def test_top_k_extremes_reduce_to_plain_draws():
    g = np.random.default_rng(2)
    logits = g.standard_normal((5, 64)) * 2
    seeds, offs = [1, 2, 3, 4, 5], [0, 1, 2, 3, 4]
    plain, _ = S.sample(logits, seeds, offs, 1.0)
    for k in (64, 100, 0, None):
        ids, _ = S.sample(logits, seeds, offs, 1.0, top_k=k)
        assert np.array_equal(ids, plain)
    ids, _ = S.sample(logits, seeds, offs, 1.0, top_k=1)
    assert np.array_equal(ids, np.argmax(logits, axis=1))
