"""The CPU oracle of TInferSampler pinned by the reference's own sampler test
(TTestInferLlmNative.SamplerDraws, tests/test.infer.llm.pas:1111-1365): the
splitmix64 draws of seed 42, the distributions of temperature, top-k (with
ties, by logit), top-p (over the whole mass, after top-k), min-p (after
top-p), NaN and -Inf never drawn, greedy cases, refused settings and the
nucleus of a 151936-token vocabulary."""
import numpy as np
import pytest

import oracle_lib as O

N = 70000


def draws(logits, n=N, **kw):
    s = O.Sampler(**kw)
    c = np.zeros(len(logits), np.int64)
    for _ in range(n):
        c[s.next(logits)] += 1
    s.close()
    return c


def near(count, share, n=N):
    return abs(count / n - share) < 0.01


L3 = np.float32([0, np.log(2), np.log(4)])
NAN, NINF = np.uint32(0x7FC00000).view(np.float32), np.uint32(0xFF800000).view(np.float32)


def test_seed_42_draws_everywhere():
    s = O.Sampler(1, 0, 1, 0, 42)
    assert [s.next(L3) for _ in range(12)] == [2, 1, 1, 1, 0, 2, 1, 2, 1, 2, 1, 2]
    a, b, c = O.Sampler(seed=42), O.Sampler(seed=42), O.Sampler(seed=43)
    sa = [a.next(L3) for _ in range(200)]
    assert sa == [b.next(L3) for _ in range(200)]
    assert sa != [c.next(L3) for _ in range(200)]


def test_splitmix64_stream():
    # Vigna's splitmix64 from state 0: the first outputs of the published
    # generator are 0xe220a8397b1dcdaf, 0x6e789e6aa1b965f4, 0x06c45d188009454f
    import ctypes as C
    st = C.c_uint64(0)
    for z in (0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F):
        assert O.lib().orc_splitmix_next(C.byref(st)) == (z >> 11) / 9007199254740992.0


def test_distributions():
    c = draws(L3, temperature=1, seed=1)
    assert near(c[0], 1 / 7) and near(c[1], 2 / 7) and near(c[2], 4 / 7)
    c = draws(L3, temperature=0.5, seed=2)
    assert near(c[0], 1 / 21) and near(c[1], 4 / 21) and near(c[2], 16 / 21)
    c = draws(L3, top_k=2, seed=3)
    assert c[0] == 0 and near(c[1], 1 / 3) and near(c[2], 2 / 3)
    assert draws(L3, top_p=0.5, seed=4)[2] == N
    c = draws(L3, top_p=0.6, seed=5)
    assert c[0] == 0 and near(c[1], 1 / 3) and near(c[2], 2 / 3)
    c = draws(L3, min_p=0.4, seed=6)
    assert c[0] == 0 and near(c[1], 1 / 3) and near(c[2], 2 / 3)
    assert draws(L3, top_k=2, top_p=0.6, seed=7)[2] == N


def test_top_p_over_the_whole_mass():
    big = np.full(1002, np.log(1e-4), np.float32)
    big[0], big[1] = 0, np.log(0.5)
    c = draws(big, top_p=0.65, seed=10)
    assert near(c[0], 2 / 3) and near(c[1], 1 / 3)


def test_top_k_ties_and_logit_order():
    c = draws(np.zeros(3, np.float32), top_k=2, seed=11)
    assert all(near(x, 1 / 3) for x in c)
    assert draws(np.float32([0, 1e-20, -50]), 1000, top_k=1, seed=15)[1] == 1000


def test_nan_and_inf():
    odd = np.float32([1, 1, NINF, NAN])
    c = draws(odd, seed=16)
    assert c[2] == 0 and c[3] == 0 and near(c[0], 0.5)
    odd = np.float32([NAN, 1, NINF, 1])
    c = draws(odd, seed=9)
    assert c[0] == 0 and c[2] == 0 and near(c[1], 0.5) and near(c[3], 0.5)


def test_top_p_before_min_p():
    l = np.log(np.float32([0.5, 0.3, 0.2])).astype(np.float32)
    c = draws(l, top_p=0.6, min_p=0.5, seed=12)
    assert c[2] == 0 and near(c[0], 0.625) and near(c[1], 0.375)


def test_top_k_beyond_the_finite_tokens():
    v = np.full(100, NINF, np.float32)
    v[0], v[7], v[50] = 0, np.log(2), np.log(4)
    c = draws(v, top_k=50, seed=13)
    assert c[0] + c[7] + c[50] == N and near(c[0], 1 / 7) and near(c[50], 4 / 7)


def test_greedy_cases():
    l = np.log(np.float32([0.5, 0.3, 0.2])).astype(np.float32)
    assert draws(l, 100, temperature=1e-310, seed=14)[0] == 100
    assert draws(L3, 100, temperature=0, seed=8)[2] == 100


def test_refused_settings():
    for kw in (dict(top_p=0), dict(top_p=1.5), dict(min_p=1), dict(top_k=-1), dict(min_p=-0.1),
               dict(temperature=float("nan"))):
        with pytest.raises(ValueError):
            O.Sampler(**kw)


def test_nucleus_of_a_real_vocabulary():
    t = 12345
    big = np.empty(151936, np.float32)
    for i in range(big.size):
        t = (t * 1103515245 + 12345) & 0x7FFFFFFF
        big[i] = (t / 0x7FFFFFFF) * 12 - 6
    m = big[O.argmax(big)]
    prob = np.exp((big.astype(np.float64) - m) / 0.7)
    prob /= prob.sum()
    # the nucleus: the largest threshold whose tokens still sum to 0.9
    order = np.sort(prob)[::-1]
    thr = order[np.searchsorted(np.cumsum(order), 0.9)]
    s = O.Sampler(0.7, 0, 0.9, 0, 77)
    got = [s.next(big) for _ in range(100)]
    assert all(prob[k] >= thr for k in got)
    assert len(set(got)) > 50
