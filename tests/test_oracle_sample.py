"""The oracle's sampling rule (the library's lq8_sample_device rule restated on
the CPU) pinned by known answers that do not restate it:

* greedy / penalty cases from the reference's own tests
  (src/generate.rs:419-545, 848-890), observed through the chosen token;
* the random stream: with equal logits every candidate weighs exactly 2^32,
  so the token is floor(n * u24 / 2^24) for n candidates, u24 the top 24 bits
  of a textbook SplitMix64 output, written out here independently;
* the distribution: chi-square of many draws against softmax(x / T),
  restricted to the top-k / nucleus support;
* GenerationConfig defaults and validation (src/generate.rs:389-417).
"""
import math

import numpy as np
import pytest

import lq8
import oracle

GOLDEN = 0x9E3779B97F4A7C15
M64 = 2**64 - 1


def splitmix64(state: int) -> int:
    """SplitMix64 (Steele, Lea, Flood 2014): one step from ``state``."""
    z = (state + GOLDEN) & M64
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M64
    return z ^ (z >> 31)


def draw(logits, n, seed=1, counts=None, **kw):
    cfg = dict(temperature=1.0, top_k=0, top_p=1.0, repetition_penalty=1.0)
    cfg.update(kw)
    return np.array([oracle.sample(logits, counts, cfg["temperature"], cfg["top_k"], cfg["top_p"],
                                   cfg["repetition_penalty"], seed, s) for s in range(n)])


def test_splitmix64_known_value():
    # the published first output of SplitMix64 seeded with 0
    assert splitmix64(0) == 0xE220A8397B1DCDAF


def test_greedy_cases_from_reference_tests():
    g = lambda x: oracle.sample(np.array(x, np.float32), None, 0.0, 0, 1.0, 1.0, 0, 0)
    assert g([1.0, 2.0, 5.0, 1.0, 0.5]) == 2
    assert g([2.0, 1.0, 0.5, 4.0, 1.0]) == 3
    assert g([1.0, 3.0, 2.0, 0.5]) == 1
    assert g([1.0, 5.0, 2.0, 4.0, 3.0]) == 1
    # top_k / top_p do not matter at temperature 0
    assert oracle.sample(np.array([1.0, 5.0, 2.0, 4.0, 3.0], np.float32), None, 0.0, 3, 0.9, 1.0, 0, 0) == 1


def test_greedy_ties_take_the_last_index():
    assert oracle.sample(np.array([1.0, 3.0, 3.0, 0.0], np.float32), None, 0.0, 0, 1.0, 1.0, 0, 0) == 2
    x = np.zeros(1000, np.float32)
    assert oracle.sample(x, None, 0.0, 0, 1.0, 1.0, 0, 0) == 999


def test_repetition_penalty_known_answers():
    s = lambda x, c, p: oracle.sample(np.array(x, np.float32), np.array(c, np.uint32), 0.0, 0, 1.0, p, 0, 0)
    # positive logits are divided: 5 -> 2.5 loses to 4
    assert s([1, 2, 3, 4, 5], [0, 0, 0, 0, 1], 2.0) == 3
    assert s([1, 2, 3, 4, 5], [0, 0, 0, 0, 1], 1.0) == 4          # penalty 1 changes nothing
    assert s([1, 2, 3, 4, 5], [0, 0, 0, 0, 0], 2.0) == 4          # nothing generated yet
    # negative logits are multiplied: -1 -> -2.5 falls below -2 (a divide would keep it on top)
    assert s([-2, -3, -1, -4], [0, 0, 1, 0], 2.5) == 0
    # a zero logit is left alone
    assert s([0.0, -0.5], [1, 0], 2.0) == 0
    # once per earlier occurrence: 4 -> 3.33 still beats 3, 4 -> 2.78 does not
    assert s([4, 3], [1, 0], 1.2) == 0
    assert s([4, 3], [2, 0], 1.2) == 1


@pytest.mark.parametrize("seed", [0, 7, 2**64 - 5])
def test_random_stream_equal_weights(seed):
    """Equal logits: candidate j sits at sorted position j (lower index first),
    every weight is 2^32 and C_j = (j + 1) 2^32, so with n candidates in the
    draw the token is floor(n * u24 / 2^24)."""
    x = np.zeros(256, np.float32)
    for step in range(40):
        u24 = splitmix64((seed + step * GOLDEN) & M64) >> 40
        assert oracle.sample(x, None, 1.0, 0, 1.0, 1.0, seed, step) == (256 * u24) >> 24, step
        # top_k 100: C_end = 100 * 2^32
        assert oracle.sample(x, None, 0.7, 100, 1.0, 1.0, seed, step) == (100 * u24) >> 24, step
    x = np.zeros(300, np.float32)
    for step in range(40):
        # nucleus 0.5 of 300 equal weights: thr = 150 * 2^32, reached at the 150th
        u24 = splitmix64((seed + step * GOLDEN) & M64) >> 40
        assert oracle.sample(x, None, 1.0, 0, 0.5, 1.0, seed, step) == (150 * u24) >> 24, step


def test_integer_weights_known_answers():
    """Two candidates z = (0, fl(-ln 2)): weights 2^32 and 2^32 * fl(exp(z_1))
    (the exponential rounded once to float, here from numpy in double), so
    C = (2^32, 2^32 + w_1) and the first candidate is drawn exactly when
    r = floor(C_end * u24 / 2^24) < 2^32."""
    x = np.array([0.0, -0.6931471805599453], np.float32)
    w1 = int(np.float32(np.exp(np.float64(x[1]))) * np.float32(2**32))
    for step in range(64):
        u24 = splitmix64((9 + step * GOLDEN) & M64) >> 40
        r = ((2**32 + w1) * u24) >> 24
        assert oracle.sample(x, None, 1.0, 0, 1.0, 1.0, 9, step) == (0 if 2**32 > r else 1), step
    # a weight below 2^-32 of the top is 0: never drawn
    x = np.array([0.0, -30.0], np.float32)
    assert set(draw(x, 200, seed=2)) == {0}


def chi2_ok(counts, probs, n):
    exp = probs * n
    stat = float(np.sum((counts - exp) ** 2 / exp))
    dof = len(probs) - 1
    # Wilson-Hilferty upper 1e-4 quantile of chi-square(dof)
    z = 3.719
    crit = dof * (1 - 2 / (9 * dof) + z * math.sqrt(2 / (9 * dof))) ** 3
    return stat < crit, stat, crit


@pytest.mark.parametrize("temperature", [1.0, 0.5, 2.0])
def test_distribution_matches_softmax(temperature):
    x = np.array([1.0, 0.2, -0.5, 2.0, 1.5, 0.0], np.float32)
    n = 12000
    toks = draw(x, n, seed=11, temperature=temperature)
    p = np.exp(x / temperature - np.max(x / temperature))
    p /= p.sum()
    ok, stat, crit = chi2_ok(np.bincount(toks, minlength=x.size), p, n)
    assert ok, (stat, crit)


def test_top_k_support_and_renormalisation():
    x = np.array([1.0, 0.2, -0.5, 2.0, 1.5, 0.0], np.float32)
    toks = draw(x, 8000, seed=3, top_k=3)
    assert set(np.unique(toks)) == {0, 3, 4}
    keep = np.array([0, 3, 4])
    p = np.exp(x[keep] - x.max())
    p /= p.sum()
    ok, stat, crit = chi2_ok(np.bincount(toks, minlength=x.size)[keep], p, toks.size)
    assert ok, (stat, crit)
    # top_k 1 is the first maximum whatever the draw
    assert set(draw(np.array([0.0, 3.0, 3.0], np.float32), 50, top_k=1)) == {1}


def test_top_k_ties_keep_lower_indices():
    assert set(draw(np.ones(8, np.float32), 400, seed=5, top_k=2)) == {0, 1}


def test_top_p_nucleus():
    probs = np.array([0.5, 0.3, 0.15, 0.05])
    x = np.log(probs).astype(np.float32)
    # 0.5 < 0.7 <= 0.8: the nucleus is {0, 1}, sampled 5:3
    toks = draw(x, 8000, seed=9, top_p=0.7)
    assert set(np.unique(toks)) == {0, 1}
    ok, stat, crit = chi2_ok(np.bincount(toks, minlength=4)[:2], probs[:2] / 0.8, toks.size)
    assert ok, (stat, crit)
    # below the first candidate's share only the first survives
    assert set(draw(x, 200, seed=9, top_p=0.45)) == {0}
    # top_p 0: the first candidate
    assert set(draw(x, 50, seed=9, top_p=0.0)) == {0}
    # top_k and top_p together: top_k 3 then 90 % of (0.5 + 0.3 + 0.15)
    toks = draw(x, 4000, seed=4, top_k=3, top_p=0.9)
    assert set(np.unique(toks)) == {0, 1, 2}


def test_seed_and_step_select_the_draw():
    x = np.array([1.0, 0.2, -0.5, 2.0, 1.5, 0.0], np.float32)
    a, b, c = draw(x, 64, seed=1), draw(x, 64, seed=1), draw(x, 64, seed=2)
    assert a.tolist() == b.tolist()
    assert a.tolist() != c.tolist()


def test_generation_config_defaults_and_validation():
    d = lq8.GenerationConfig()
    assert (d.max_new_tokens, d.temperature, d.top_k, d.top_p, d.repetition_penalty) == (100, 0.0, 0, 1.0, 1.0)
    c = lq8.GenerationConfig.new(50, 0.8, 10, 0.9, 1.2)
    assert c.max_new_tokens == 50 and c.temperature == pytest.approx(0.8)
    for bad in [(50, -0.1, 10, 0.9, 1.2), (50, 0.8, 10, 1.5, 1.2), (50, 0.8, 10, 0.9, 0.5),
                (50, 0.8, 10, -0.1, 1.2)]:
        with pytest.raises(lq8.InvalidArgument):
            lq8.GenerationConfig.new(*bad)
