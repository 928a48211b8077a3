"""The CPU oracle's stochastic sampler (the reference's sample_logits,
cpu_lightspark.py:706-726) against numpy running the reference's own steps,
numpy's Generator.choice, and closed-form special cases."""
import numpy as np
import pytest

import oracle


class Args:
    def __init__(self, temperature=0.7, top_k=40, top_p=0.9, repetition_penalty=1.08, argmax=False):
        self.temperature, self.top_k, self.top_p = temperature, top_k, top_p
        self.repetition_penalty, self.argmax = repetition_penalty, argmax


def numpy_sampler(logits, generated, args, u):
    """cpu_lightspark.py:706-726 as the reference runs it in numpy, with
    generator.choice(ids, p) replaced by its definition given the draw u
    (test_choice_restatement_matches_numpy pins that replacement)."""
    values = np.array(logits, dtype=np.float32, copy=True).reshape(-1)
    if generated and args.repetition_penalty != 1.0:
        ids = np.array(sorted(set(generated)), dtype=np.int64)
        repeated = values[ids]
        values[ids] = np.where(repeated > 0, repeated / np.float32(args.repetition_penalty),
                               repeated * np.float32(args.repetition_penalty))
    values /= np.float32(args.temperature)
    count = min(args.top_k, values.size)
    ids = np.argpartition(-values, count - 1)[:count]
    ids = ids[np.argsort(-values[ids])]
    selected = values[ids]
    selected -= selected.max()
    probabilities = np.exp(selected, dtype=np.float32)
    probabilities /= probabilities.sum(dtype=np.float32)
    if args.top_p < 1.0:
        probabilities[(np.cumsum(probabilities) - probabilities) >= args.top_p] = 0
        probabilities /= probabilities.sum(dtype=np.float32)
    cdf = probabilities.astype(np.float64).cumsum()
    cdf /= cdf[-1]
    return int(ids[np.searchsorted(cdf, u, side="right")]), ids, probabilities, cdf, values


def test_choice_restatement_matches_numpy():
    # Generator.choice(a, p=p) draws one random() and searches the normalised
    # float64 cdf of p (side="right"); the same seed gives the same element
    rng = np.random.default_rng(123)
    for trial in range(300):
        k = int(rng.integers(1, 64))
        p = rng.random(k).astype(np.float32)
        p[rng.random(k) < 0.3] = 0
        if p.sum() == 0:
            p[0] = 1
        p /= p.sum(dtype=np.float32)
        ids = rng.permutation(1000)[:k]
        a = np.random.default_rng(trial).choice(ids, p=p)
        cdf = p.astype(np.float64).cumsum()
        cdf /= cdf[-1]
        u = np.random.default_rng(trial).random()
        assert a == ids[np.searchsorted(cdf, u, side="right")]


@pytest.mark.parametrize("n", list(range(1, 40)) + [63, 64, 65, 100, 127, 128, 129, 136, 200, 256, 257,
                                                   1000, 2047, 2048, 4096])
def test_pairwise_sum_is_numpys_float32_sum(n):
    rng = np.random.default_rng(n)
    a = (rng.random(n) * 10 ** rng.uniform(-3, 3, n)).astype(np.float32)
    assert oracle.pairwise_sum_f32(a).view(np.uint32) == a.sum(dtype=np.float32).view(np.uint32)


def test_sampler_matches_reference_steps_in_numpy():
    rng = np.random.default_rng(7)
    boundary = ties = 0
    for trial in range(400):
        n = int(rng.choice([50, 1000, 151936]))
        logits = (rng.standard_normal(n) * rng.uniform(0.5, 8)).astype(np.float32)
        generated = list(rng.integers(0, n, int(rng.integers(0, 30))))
        top_k = int(rng.integers(1, 80)) if trial % 8 else int(rng.choice([200, 1000, 2048]))
        args = Args(temperature=float(rng.uniform(0.3, 1.5)), top_k=top_k,
                    top_p=float(rng.choice([1.0, 0.9, 0.5, 0.99])),
                    repetition_penalty=float(rng.choice([1.0, 1.08, 1.3])))
        u = float(rng.random())
        want, ids, probs, cdf, values = numpy_sampler(logits, generated, args, u)
        got, gids, gprobs = oracle.sample_token(logits, generated, args.repetition_penalty, args.temperature,
                                                args.top_k, args.top_p, u)
        # numpy's argsort is not stable: equal values may come in either
        # order there; the oracle ranks them by index
        np.testing.assert_array_equal(values[gids], values[ids])
        differ = gids != ids
        ties += int(differ.sum())
        for v in np.unique(values[gids][differ]):
            run = gids[values[gids] == v]
            assert np.all(np.diff(run) > 0)
        # probabilities differ from numpy's only through exp (< 2 ulp each)
        np.testing.assert_allclose(gprobs, probs, rtol=3e-6, atol=1e-12)
        if got != want and values[got] != values[want]:     # (a tied value is the same draw)
            boundary += 1
            assert np.min(np.abs(cdf - u)) < 1e-5, (trial, got, want)
    assert boundary <= 2 and ties <= 20


def test_sampler_special_cases():
    x = np.array([0.5, 3.0, -2.0, 2.9, 1.0], np.float32)
    # top_k = 1 is argmax for every draw
    for u in (0.0, 0.5, 0.999999):
        assert oracle.sample_token(x, [], 1.0, 0.7, 1, 0.9, u)[0] == 1
    # a tiny top_p keeps only the most likely token
    assert oracle.sample_token(x, [], 1.0, 0.7, 5, 1e-9, 0.999)[0] == 1
    # the penalty divides a positive logit (3.0 -> 1.5 < 2.9) and multiplies a
    # negative one; a repeated id counts once
    tok, ids, _ = oracle.sample_token(x, [1, 1, 1], 2.0, 1.0, 5, 1.0, 0.0)
    assert list(ids) == [3, 1, 4, 0, 2] and tok == 3
    _, ids, probs = oracle.sample_token(x, [2], 2.0, 1.0, 5, 1.0, 0.0)
    assert ids[-1] == 2
    np.testing.assert_allclose(probs[-1], np.exp(np.float32(-4.0) - np.float32(3.0)) / np.exp(
        x[[1, 3, 4, 0]] - np.float32(3.0)).sum() / (1 + np.exp(np.float32(-7.0)) / np.exp(
        x[[1, 3, 4, 0]] - np.float32(3.0)).sum()), rtol=1e-5)
    # equal values rank by index; u just below a cdf step picks the earlier id
    y = np.array([1.0, 2.0, 2.0, 0.0], np.float32)
    tok, ids, probs = oracle.sample_token(y, [], 1.0, 1.0, 4, 1.0, 0.0)
    assert list(ids) == [1, 2, 0, 3] and tok == 1
    cdf = np.cumsum(probs.astype(np.float64))
    cdf /= cdf[-1]
    assert oracle.sample_token(y, [], 1.0, 1.0, 4, 1.0, np.nextafter(cdf[0], 0))[0] == 1
    assert oracle.sample_token(y, [], 1.0, 1.0, 4, 1.0, cdf[0])[0] == 2
