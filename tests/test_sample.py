"""The oracle's LmHead::sample (aideen-backbone/src/lm_head.rs:78-168) pinned by what the
mathematics fixes.  The reference has no test of its own for sample and draws its uniform from
thread_rng; here the draw r is an argument (rng.gen::<f32>() makes 24-bit values in [0, 1)).

- temperature <= 0: the arg-max (last maximum) of the penalised logits; a temperature in
  (0, 1e-4] divides and samples (two tied maxima then split the draws at 1/2);
- top_k = 1: the first maximum (the sorted list is stable, ties in index order) for every draw;
- inverse CDF: stratified draws r_j = (j + 1/2)/N land on each token about N p times (float64
  softmax), in descending order of p;
- the temperature and the penalty act on the logits only: sample(x, T, ctx, pen) equals sample of
  the penalised and divided logits at T = 1 with no context;
- top-k and top-p keep the sets the float64 sorted sums give, with frequencies of the renormalised
  probabilities;
- a NaN or infinite logit: the arg-max of the row as given (the penalty not applied).
"""
import numpy as np
import pytest

F32 = np.float32


def draws(rng, n):
    return (rng.integers(0, 1 << 24, size=n) * 2.0 ** -24).astype(F32)


def penalise(x, ctx, pen):
    """lm_head.rs:81-99 in numpy: each distinct context token once."""
    y = np.array(x, F32)
    if abs(pen - 1.0) > 1e-4 and len(ctx):
        for t in dict.fromkeys(int(v) for v in ctx):
            if 0 <= t < y.size:
                y[t] = y[t] * F32(pen) if y[t] < 0 else y[t] / F32(pen)
    return y


def softmax64(x):
    z = np.asarray(x, np.float64)
    e = np.exp(z - z.max())
    return e / e.sum()


def test_greedy_is_penalised_last_max(oracle_lib):
    rng = np.random.default_rng(1)
    x = rng.standard_normal(300).astype(F32)
    x[[17, 200]] = x.max() + 1  # a tied maximum: the last one wins
    ctx = [200, 5, 5, 9]
    for T in (0.0, -1.0):
        t = oracle_lib.lm_sample(x, [], T, 0.9, 40, 1.0, 0.3)[0]
        assert t == 200
        y = penalise(x, ctx, 1.5)
        t = oracle_lib.lm_sample(x, ctx, T, 0.9, 40, 1.5, 0.3)[0]
        assert t == int(np.flatnonzero(y == y.max())[-1]) == 17


def test_tiny_positive_temperature_divides_and_samples(oracle_lib):
    x = np.zeros(50, F32)
    x[[7, 31]] = 3.0
    # greedy (T <= 0) takes the last maximum; T = 5e-5 divides, the two maxima carry p = 1/2 each
    assert oracle_lib.lm_sample(x, [], 0.0, 1.0, 0, 1.0, 0.2)[0] == 31
    assert oracle_lib.lm_sample(x, [], 5e-5, 1.0, 0, 1.0, 0.2)[0] == 7
    assert oracle_lib.lm_sample(x, [], 5e-5, 1.0, 0, 1.0, 0.7)[0] == 31


def test_top1_is_first_max(oracle_lib):
    rng = np.random.default_rng(2)
    x = rng.standard_normal(1000).astype(F32)
    x[[40, 41, 900]] = x.max() + 0.5
    for T in (0.7, 1.0, 2.0):
        for r in draws(rng, 20):
            assert oracle_lib.lm_sample(x, [], T, 1.0, 1, 1.0, r)[0] == 40


def test_zero_draw_takes_the_top_item(oracle_lib):
    rng = np.random.default_rng(3)
    x = rng.standard_normal(500).astype(F32)
    assert oracle_lib.lm_sample(x, [], 1.3, 0.9, 0, 1.0, 0.0)[0] == int(np.argmax(x))


def test_inverse_cdf(oracle_lib):
    rng = np.random.default_rng(4)
    x = rng.standard_normal(40).astype(F32)
    p = softmax64(x)
    N = 4000
    toks = [oracle_lib.lm_sample(x, [], 1.0, 1.0, 0, 1.0, F32((j + 0.5) / N))[0] for j in range(N)]
    counts = np.bincount(toks, minlength=x.size)
    assert np.abs(counts - N * p).max() <= 2.0
    # the draws walk the tokens in descending probability order
    seen = list(dict.fromkeys(toks))
    order = [int(i) for i in np.argsort(-p, kind="stable") if counts[i] > 0]
    assert seen == order


def test_temperature_and_penalty_act_on_the_logits(oracle_lib):
    rng = np.random.default_rng(5)
    x = (2.0 * rng.standard_normal(800)).astype(F32)
    ctx = rng.integers(0, 800, size=30).tolist()
    for T, pen, top_p, top_k in ((0.8, 1.1, 0.9, 40), (1.7, 1.3, 1.0, 0), (0.5, 0.9, 0.5, 300)):
        y = penalise(x, ctx, pen) / F32(T)
        for r in draws(rng, 30):
            a = oracle_lib.lm_sample(x, ctx, T, top_p, top_k, pen, r)[0]
            b = oracle_lib.lm_sample(y, [], 1.0, top_p, top_k, 1.0, r)[0]
            assert a == b


@pytest.mark.parametrize("top_k,top_p", [(20, 1.0), (0, 0.6), (20, 0.6), (300, 0.3)])
def test_top_k_top_p_sets_and_frequencies(oracle_lib, top_k, top_p):
    rng = np.random.default_rng(6)
    x = (1.5 * rng.standard_normal(500)).astype(F32)
    p = softmax64(x)
    order = np.argsort(-p, kind="stable")
    kept = order[:top_k] if 0 < top_k < x.size else order
    if 0 < top_p < 1:
        cum = np.cumsum(p[kept])
        cut = int(np.flatnonzero(cum > top_p)[0]) + 1 if (cum > top_p).any() else kept.size
        kept = kept[:cut]
    q = p[kept] / p[kept].sum()
    N = 3000
    toks = []
    for j in range(N):
        toks.append(oracle_lib.lm_sample(x, [], 1.0, top_p, top_k, 1.0, F32((j + 0.5) / N))[0])
    assert set(toks) <= set(kept.tolist())
    counts = np.array([toks.count(int(i)) for i in kept])
    assert np.abs(counts - N * q).max() <= 2.0


def test_nonfinite_logits_take_the_argmax_of_the_row_as_given(oracle_lib):
    rng = np.random.default_rng(7)
    x = rng.standard_normal(100).astype(F32)
    ctx = [3, 50, 99]
    y = x.copy()
    y[[10, 60]] = np.nan  # the fold restarts after the last NaN: the last maximum after index 60
    want = 61 + int(np.flatnonzero(y[61:] == y[61:].max())[-1])
    assert oracle_lib.lm_sample(y, ctx, 0.8, 0.9, 40, 1.3, 0.5)[0] == want
    assert oracle_lib.argmax(y) == want
    y = x.copy()
    y[[20, 70]] = np.inf
    assert oracle_lib.lm_sample(y, ctx, 0.8, 0.9, 40, 1.3, 0.5)[0] == 70
    y = np.full(100, -np.inf, F32)
    assert oracle_lib.lm_sample(y, [], 0.8, 0.9, 0, 1.0, 0.5)[0] == 99


def test_conditioning_flags_a_draw_on_a_boundary(oracle_lib):
    """The conditioning the device parity tests rely on: a draw on a running-sum boundary, two
    decisive items with logits an ulp apart, or a running sum at top_p reads below 1; a draw in the
    middle of an item's interval reads far above; the kept list's length comes with it."""
    x = np.array([2.0, 1.0, 0.0, -1.0], F32)
    p = softmax64(x)
    assert oracle_lib.lm_sample(x, [], 1.0, 1.0, 0, 1.0, F32(p[0]))[1] < 1.0
    t, cond, kept = oracle_lib.lm_sample(x, [], 1.0, 1.0, 0, 1.0, F32(p[0] / 2))
    assert (t, kept) == (0, 4) and cond > 100.0
    y = np.array([2.0, np.nextafter(F32(2.0), F32(3.0)), 0.0], F32)
    assert oracle_lib.lm_sample(y, [], 1.0, 1.0, 0, 1.0, F32(0.3))[1] < 1.0
    z = np.array([2.0, 2.0, 0.0], F32)  # an exact tie is the same on every device
    assert oracle_lib.lm_sample(z, [], 1.0, 1.0, 0, 1.0, F32(0.3))[1] > 1.0
    assert oracle_lib.lm_sample(x, [], 1.0, F32(p[0]), 0, 1.0, F32(0.3))[1] < 1.0
    assert oracle_lib.lm_sample(x, [], 1.0, F32(p[0] + 0.01), 0, 1.0, F32(0.3))[2] == 2
