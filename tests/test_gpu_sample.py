"""LmHead::sample (lm_head.rs:78-168) on the device against the oracle (needs an MI355X).

The reference draws its uniform from thread_rng; the device takes the draw as an argument, so each
draw is compared token for token.  The device computes its own probabilities (exp rounded once
from double, its own summation order), so a draw whose running sum lies within rounding of a
boundary can go either way: the oracle reports each decision's conditioning (orc_lm_sample), and
every decision with conditioning >= 1 must give the oracle's token; at least 90% of the draws of
each group must be such decisions, so the comparison cannot pass by excluding them.
"""
import dataclasses

import numpy as np
import pytest

from aideen_amd import synth
from test_gpu_parity import _small, log, make

pytestmark = pytest.mark.gpu

F32 = np.float32

# (temperature, top_p, top_k, repetition penalty): the reference binaries' own choice (train.rs,
# benchmark.rs: 0.8, 0.9, 40, 1.1), no cut at all, a top-p cut alone, top-k beyond the sorted-list
# bound with and without top-p, a temperature in (0, 1e-4], and T = 1 exactly
GROUPS = [
    (0.8, 0.9, 40, 1.1),
    (1.0, 1.0, 0, 1.0),
    (0.7, 0.95, 0, 1.3),
    (1.5, 0.5, 3000, 1.0),
    (1.2, 1.0, 5000, 1.2),
    (0.5, 0.3, 0, 1.0),
    (5e-5, 0.9, 40, 1.1),
    (1.0, 0.9, 100, 1.0),
]


def draws(rng, n):
    return (rng.integers(0, 1 << 24, size=n) * 2.0 ** -24).astype(F32)


def rows_for(rng, V, n, sigma):
    x = (sigma * rng.standard_normal((n, V))).astype(F32)
    # exact ties among the large logits (duplicated rows of W_lm give equal logits)
    for i in range(n):
        top = np.argsort(-x[i])[:8]
        x[i, top[1::2]] = x[i, top[0::2]]
    return x


def compare(oracle_lib, x, ctx, uni, got, T, top_p, top_k, pen, label):
    """Every conditioned draw equal.  Returns the counts (draws, conditioned) for kept lists of at
    most 2048 items and for longer ones."""
    n = [0, 0]
    ok = [0, 0]
    for i in range(x.shape[0]):
        t, cond, kept = oracle_lib.lm_sample(x[i], ctx[i], T, top_p, top_k, pen, uni[i])
        k = int(kept > 2048)
        n[k] += 1
        if cond >= 1.0:
            ok[k] += 1
            assert got[i] == t, f"{label} row {i}: device {got[i]}, oracle {t} (cond {cond:.3g}, r {uni[i]})"
    log(f"{label}: conditioned and equal: {ok[0]} of {n[0]} draws with short kept lists, {ok[1]} of {n[1]} with long")
    return n, ok


@pytest.fixture(scope="module")
def backend():
    mc, _ = _small(d=64, H=1, V=300, N=1)
    be = make(mc, 4, 4)
    yield be
    be.close()


@pytest.mark.parametrize("V", [50257, 2048, 300])
@pytest.mark.parametrize("grp", GROUPS, ids=lambda g: "T{}-p{}-k{}-pen{}".format(*g))
def test_lm_sample_matches_oracle(oracle_lib, backend, V, grp):
    T, top_p, top_k, pen = grp
    rng = np.random.default_rng(V + int(1000 * T) + top_k)
    n = 48 if V > 4096 else 96
    tot, tok = np.zeros(2, int), np.zeros(2, int)
    for sigma in (0.5, 2.0, 6.0):
        x = rows_for(rng, V, n, sigma)
        ctx = [rng.integers(0, V, size=int(rng.integers(0, 40))).tolist() for _ in range(n)]
        uni = draws(rng, n)
        uni[0] = 0.0
        got = backend.lm_sample(x, uni, temperature=T, top_p=top_p, top_k=top_k, repetition_penalty=pen,
                                context=ctx)
        c, o = compare(oracle_lib, x, ctx, uni, got, T, top_p, top_k, pen, f"V={V} {grp} sigma={sigma}")
        tot += c
        tok += o
    # at least 90% of the draws conditioned where the kept list is at most 2048 long, a quarter
    # where it is longer (over tens of thousands of nearly equal probabilities the reference's own
    # float running sums move many draws across a boundary: those are its rounding)
    assert tok[0] >= 0.9 * tot[0], f"{grp}: too few conditioned draws among the short kept lists"
    assert tok[1] >= 0.25 * tot[1], f"{grp}: too few conditioned draws among the long kept lists"


def test_lm_sample_edge_rows(oracle_lib, backend):
    """NaN and infinite logits (the arg-max of the row as given), no finite logit, uniform logits
    (every probability equal: the list in index order), one token, top_k >= V and V - 1, a top_p
    below the largest probability, NaN temperature (no scaling), temperature <= 0 (the penalised
    arg-max), a draw of 0 and the largest draw."""
    rng = np.random.default_rng(11)
    V = 5000
    base = rng.standard_normal(V).astype(F32)
    rows, params = [], []

    def add(x, T=0.8, top_p=0.9, top_k=40, pen=1.1, r=0.5, ctx=(1, 2, 3)):
        rows.append((np.asarray(x, F32), list(ctx), F32(r)))
        params.append((T, top_p, top_k, pen))

    y = base.copy(); y[[5, 4000]] = np.nan; add(y)
    y = base.copy(); y[[9, 99]] = np.inf; add(y)
    add(np.full(V, -np.inf, F32))
    y = base.copy(); y[7] = -np.inf; add(y, top_k=0, top_p=1.0)
    for r in (0.0, 0.25, 0.5, 1.0 - 2.0 ** -24):
        add(np.zeros(V, F32), top_k=0, top_p=1.0, r=r, ctx=())
    add(base, top_k=V), add(base, top_k=V - 1), add(base, top_k=V + 5, top_p=1.0)
    add(base, top_p=1e-6), add(base, T=float("nan")), add(base, T=0.0), add(base, T=-2.0, pen=1.5)
    add(base, r=1.0 - 2.0 ** -24, top_k=0, top_p=0.999)
    # one row per call: the parameters differ from row to row
    for i, ((x, ctx, r), (T, top_p, top_k, pen)) in enumerate(zip(rows, params)):
        got = backend.lm_sample(x[None, :], np.array([r]), temperature=T, top_p=top_p, top_k=top_k,
                                repetition_penalty=pen, context=[ctx])[0]
        t, cond, kept = oracle_lib.lm_sample(x, ctx, T, top_p, top_k, pen, r)
        log(f"edge row {i}: device {got}, oracle {t}, cond {cond:.3g}, kept {kept}")
        if cond >= 1.0:
            assert got == t, f"edge row {i}"
    one = backend.lm_sample(np.array([[0.3]], F32), np.array([0.7], F32), temperature=0.8, top_p=0.9, top_k=40)
    assert one[0] == 0


def first_difference(got, ref, cond, label):
    """The steps compared: a sequence's tokens equal the oracle's up to its first difference, which
    must fall on a draw within rounding of a boundary (after it the contexts differ)."""
    diff = np.flatnonzero(got != ref)
    if diff.size == 0:
        return got.size
    j = int(diff[0])
    assert cond[j] < 1.0, f"{label}: step {j} differs (device {got[j]}, oracle {ref[j]}, cond {cond[j]:.3g})"
    return j


def _decode_model(V=600):
    mc, w = _small(d=128, H=4, V=V, N=1, max_iters=10, eps=0.0, win_sigma=3.0)
    w["anchor"] = (w["anchor"] * np.float32(0.02)).astype(np.float32)
    return mc, w


@pytest.mark.parametrize("grp", [(0.8, 0.9, 40, 1.1), (1.0, 1.0, 0, 1.0), (0.6, 0.8, 0, 1.3)],
                         ids=lambda g: "T{}-p{}-k{}-pen{}".format(*g))
def test_decode_sample_matches_oracle(oracle_lib, grp):
    """Trainer::generate with LmHead::sample: each sequence's tokens equal the oracle's up to a
    first difference on a draw within rounding of a boundary (after it the contexts differ), over
    at least 75% of the steps; the draws change the tokens against greedy decoding."""
    T, top_p, top_k, pen = grp
    mc, w = _decode_model()
    B, T0, n_new, ctx_len = 4, 9, 24, 6
    prompt = synth.make_tokens("uniform", B, T0, mc.V, seed=12)
    rng = np.random.default_rng(21)
    uni = draws(rng, B * n_new).reshape(B, n_new)
    ref, cond = oracle_lib.Oracle(mc, w).decode_sample(prompt, n_new, ctx_len, T, top_p, top_k, pen, uni)
    be = make(mc, B, 1)
    be.upload_weights(w)
    got = be.decode_sample(prompt, n_new, ctx_len, temperature=T, top_p=top_p, top_k=top_k,
                           repetition_penalty=pen, uniforms=uni)
    greedy = be.decode_greedy(prompt, n_new, ctx_len, repetition_penalty=pen)
    be.close()
    compared = sum(first_difference(got[b], ref[b], cond[b], f"sequence {b}") for b in range(B))
    log(f"decode sample {grp}: {compared} of {B * n_new} steps compared, {len(set(ref.ravel().tolist()))} distinct tokens")
    assert compared >= 0.75 * B * n_new
    assert not np.array_equal(ref, greedy)


def test_c2_decode_sample(oracle_lib):
    """C2 (d=512, H=8, V=50257, N=16) on the token-sensitive weights: a 24-token sampled decode
    from the 256 tokens with the reference binaries' sampling (0.8, 0.9, 40, 1.1), token for token
    (a first difference only on a draw within rounding of a boundary, after at least 12 steps)."""
    p = synth.PRESETS["C2"]
    mc = dataclasses.replace(p["model"], max_iters=10, eps=0.0)
    w = synth.make_token_sensitive_weights(mc)
    toks = synth.make_tokens(p["tokens"], p["B"], p["T"], mc.V, seed=1)
    uni = draws(np.random.default_rng(5), 24).reshape(1, 24)
    ref, cond = oracle_lib.Oracle(mc, w).decode_sample(toks, 24, 256, 0.8, 0.9, 40, 1.1, uni, nthreads=16)
    be = make(mc, 1, p["T"])
    be.upload_weights(w)
    got = be.decode_sample(toks, 24, 256, temperature=0.8, top_p=0.9, top_k=40, repetition_penalty=1.1,
                           uniforms=uni)
    be.close()
    upto = first_difference(got[0], ref[0], cond[0], "C2")
    log(f"C2 decode sample: {upto} of 24 steps equal, {len(set(ref.ravel().tolist()))} distinct tokens")
    assert upto >= 12


@pytest.mark.parametrize("grp", [(0.8, 0.9, 40, 1.1), (1.0, 1.0, 0, 1.5)], ids=lambda g: "T{}-p{}-k{}-pen{}".format(*g))
def test_memory_decode_sample_matches_oracle(oracle_lib, grp):
    """The fixed-history form of Trainer::generate (trainer.rs:4395-4400, 677-735) with
    LmHead::sample: the memory primed over the prompt, each step the last token's solve with the
    memory's history context, then the draw; token for token up to a first difference on a draw
    within rounding of a boundary."""
    from test_gpu_memory import mem_model
    from aideen_amd.backend import GpuDeqBackend
    T, top_p, top_k, pen = grp
    mc, w = mem_model(128, 4, 400, max_iters=6, eps=0.0)
    B, T0, n_new, ctx_len = 3, 7, 9, 5
    prompt = synth.make_tokens("uniform", B, T0, mc.V, seed=14)
    uni = draws(np.random.default_rng(31), B * n_new).reshape(B, n_new)
    ref, cond = oracle_lib.Oracle(mc, w).decode_sample(prompt, n_new, ctx_len, T, top_p, top_k, pen, uni)
    be = GpuDeqBackend(mc, B, T0)
    be.upload_weights(w)
    got = be.decode_sample(prompt, n_new, ctx_len, temperature=T, top_p=top_p, top_k=top_k, repetition_penalty=pen,
                           uniforms=uni, max_iters=6, eps=0.0)
    greedy = be.decode_greedy(prompt, n_new, ctx_len, max_iters=6, eps=0.0, repetition_penalty=pen)
    be.close()
    compared = sum(first_difference(got[b], ref[b], cond[b], f"memory sequence {b}") for b in range(B))
    log(f"memory decode sample {grp}: {compared} of {B * n_new} steps compared")
    assert compared >= 0.75 * B * n_new
    assert not np.array_equal(ref, greedy)
