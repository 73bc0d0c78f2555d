"""Seeded random configurations against the oracle (needs an MI355X).

Each case draws a width, slot count, vocabulary, carrier, flag set (init rule, score clamp,
anchor-excluding RMS, residual norm, W_in orientation, selective carrier, q/k bias), GEMM
arithmetic, Anderson depth, batch shape, tolerance and iteration cap, so that the kernel paths
chosen by size (few-token attention inside W_o, the fixed-iteration update inside Q|K|V, the pool
inside the last update, skinny and tiled products, per-step and matrix-form scans) meet every
switch of the forward spec (fixed_point_memory_reasoning.rs:1300-1486) in combinations no
hand-written case lists.  Every output of every token is compared with the oracle on the
token-sensitive weights (the carrier's outputs against the oracle's scan of the GPU's own h*, as
everywhere: the scan is a long recurrence that would otherwise compound h*'s own tolerance).  With Anderson mixing the tolerance is 0 (the residual is not
monotone, so an exit near eps can move by two iterations; every iteration then runs), as it is
in the fixed-iteration cases.  Under that mixing a token whose oracle result itself moves by a
twentieth of the bar when a few values of each input row change by one ulp is ill-conditioned
(the last steps' Gram matrices are nearly singular): such tokens, at most 10%, are held to 50
times that response instead.
"""
import dataclasses

import numpy as np
import pytest

from aideen_amd import synth
from aideen_amd.backend import GpuDeqBackend
from test_gpu_parity import assert_forward_parity, log

pytestmark = pytest.mark.gpu

ALL = ("h_star", "pooled", "logits", "argmax", "iters", "converged", "scan_y", "scan_state")


COND_KEYS = ("h_star", "pooled", "logits")


def ulp_response(oracle_lib, mc, w, toks, ref):
    """Per token and output, how far the oracle's own result moves when a few values of every
    embedding row move by one ulp, the largest over four such changes ([B, T] arrays): with
    Anderson mixing at tolerance 0 the last steps' Gram matrices are nearly singular and some
    tokens' coefficients are set by rounding, so two correct fp32 forwards that round differently
    can disagree beyond the bar.  The response depends on the direction of the change, hence
    several."""
    d = mc.d
    probes = ((slice(0, 8), np.inf), (slice(d - 8, d), -np.inf), (slice(d // 2, d // 2 + 8), np.inf),
              (slice(0, d, 16), -np.inf))
    B, T = toks.shape
    resp = {k: np.zeros((B, T)) for k in COND_KEYS}
    for cols, to in probes:
        w2 = dict(w)
        e = np.array(w["embed"], dtype=np.float32, copy=True)
        e[:, cols] = np.nextafter(e[:, cols], np.float32(to))
        w2["embed"] = e
        ref2 = oracle_lib.Oracle(mc, w2).forward(toks, want_scan=False, nthreads=16)
        for k in COND_KEYS:
            resp[k] = np.maximum(resp[k], np.abs(ref[k] - ref2[k]).reshape(B, T, -1).max(axis=2))
    return resp


def check(oracle_lib, mc, w, toks, got, ctx):
    o = oracle_lib.Oracle(mc, w)
    ref = o.forward(toks, want_scan=False, nthreads=16)
    fwd = {k: v for k, v in got.items() if not k.startswith("scan")}
    ill = np.zeros(toks.shape, dtype=bool)
    if mc.anderson_m >= 3:
        resp = ulp_response(oracle_lib, mc, w, toks, ref)
        for k in COND_KEYS:
            ill |= resp[k] > 0.05 * 1e-3
    if ill.any():
        # tokens whose oracle result moves by a twentieth of the bar under a one-ulp input change:
        # at most 10% of them, each within 50 times that response; every other token at the bar
        log(f"{ctx}: {int(ill.sum())} of {ill.size} tokens ill-conditioned under the Anderson mix "
            f"(oracle h* moves by up to {resp['h_star'].max():.2e} under one ulp)")
        assert ill.mean() <= 0.10, f"{ctx}: {ill.mean():.3f} of the tokens ill-conditioned"
        for k in COND_KEYS:
            B, T = toks.shape
            dif = np.abs(got[k] - ref[k]).reshape(B, T, -1).max(axis=2)[ill]
            lim = 1e-3 + 1e-4 * np.abs(ref[k]).reshape(B, T, -1).max(axis=2)[ill] + 50 * resp[k][ill]
            assert (dif <= lim).all(), f"{ctx}: {k} beyond 50x the oracle's one-ulp response"
        assert_forward_parity({k: v[~ill] for k, v in fwd.items()}, {k: v[~ill] for k, v in ref.items()}, ctx)
    else:
        assert_forward_parity(fwd, ref, ctx)
    for b in range(toks.shape[0]):
        y, st = o.scan(got["h_star"][b])
        np.testing.assert_allclose(got["scan_y"][b], y, rtol=1e-4, atol=1e-3, err_msg=f"{ctx}: scan_y[{b}]")
        np.testing.assert_allclose(got["scan_state"][b], st, rtol=1e-4, atol=1e-3, err_msg=f"{ctx}: scan_state[{b}]")


def draw(seed):
    rng = np.random.default_rng(1000 + seed)
    d = int(rng.choice([64, 128, 192, 256]))
    H = int(rng.choice([1, 2, 3, 4, 5, 8]))
    V = int(rng.choice([257, 500, 1000]))
    N = int(rng.choice([1, 4, 16]))
    flags = 0
    for f in (synth.F_WIN_TRANSPOSED, synth.F_SCORE_CLAMP4, synth.F_RMS_EXCL_ANCHOR, synth.F_INIT_SIGNAL_RMS,
              synth.F_SCAN_SELECTIVE):
        if rng.random() < 0.4:
            flags |= f
    flags |= int(rng.choice([0, synth.F_RESID_L2, synth.F_RESID_RELRMS]))
    flags |= int(rng.choice([0, 0, synth.F_GEMM_BF16X3, synth.F_GEMM_FP32]))
    m = int(rng.choice([0, 0, 0, 3, 5]))
    few = rng.random() < 0.5
    B, T = ((int(rng.integers(1, 3)), int(rng.integers(1, 3))) if few else
            (int(rng.integers(1, 4)), int(rng.integers(20, 120))))
    eps = 0.0 if (m > 0 or rng.random() < 0.4) else 1e-4
    max_iters = int(rng.choice([2, 5, 9])) if eps == 0.0 else 20
    mc = synth.ModelConfig(d=d, H=H, V=V, N=N, r=32, flags=flags, anderson_m=m, eps=eps, max_iters=max_iters,
                           qk_bias=bool(rng.random() < 0.3))
    return mc, B, T


@pytest.mark.parametrize("seed", range(24))
def test_random_config_matches_oracle(oracle_lib, seed):
    mc, B, T = draw(seed)
    log(f"random config {seed}: {mc} B={B} T={T}")
    w = synth.make_token_sensitive_weights(mc, seed=seed)
    toks = synth.make_tokens("uniform", B, T, mc.V, seed=seed)
    be = GpuDeqBackend(mc, B, T)
    be.upload_weights(w)
    got = be.forward(toks, want=ALL)
    be.close()
    check(oracle_lib, mc, w, toks, got, f"random config {seed}")
    if mc.eps == 0.0:
        assert (got["iters"] == mc.max_iters).all()


def draw_large(seed):
    """At least 1024 tokens and a vocabulary of at least 512: the persistent 256 x 256 tiles of
    every product (pre-split W_o and LM-head operands), the many-token update, Anderson's one- or
    two-pass mixing, and the per-step or matrix-form carrier scan."""
    rng = np.random.default_rng(2000 + seed)
    d = int(rng.choice([128, 256, 512]))
    H = int(rng.choice([2, 4, 8]))
    V = int(rng.choice([600, 1500, 2100]))
    N = int(rng.choice([4, 16]))
    flags = synth.F_SCAN_SELECTIVE if rng.random() < 0.6 else 0
    for f in (synth.F_SCORE_CLAMP4, synth.F_RMS_EXCL_ANCHOR, synth.F_INIT_SIGNAL_RMS, synth.F_WIN_TRANSPOSED):
        if rng.random() < 0.3:
            flags |= f
    flags |= int(rng.choice([0, synth.F_RESID_L2]))
    m = int(rng.choice([0, 0, 3, 5]))
    B = int(rng.choice([1, 2, 4]))
    T = int(rng.integers(1024, 1600)) // B
    eps = 0.0 if m > 0 else 1e-4
    max_iters = 7 if eps == 0.0 else 20
    mc = synth.ModelConfig(d=d, H=H, V=V, N=N, r=32, flags=flags, anderson_m=m, eps=eps, max_iters=max_iters,
                           qk_bias=bool(rng.random() < 0.3))
    return mc, B, T


@pytest.mark.parametrize("seed", range(6))
def test_random_large_config_matches_oracle(oracle_lib, seed):
    mc, B, T = draw_large(seed)
    log(f"random large config {seed}: {mc} B={B} T={T}")
    w = synth.make_token_sensitive_weights(mc, seed=seed)
    toks = synth.make_tokens("zipf", B, T, mc.V, seed=seed)
    be = GpuDeqBackend(mc, B, T)
    be.upload_weights(w)
    got = be.forward(toks, want=ALL)
    be.close()
    check(oracle_lib, mc, w, toks, got, f"random large config {seed}")


def draw_wide(seed):
    """Rows of 1024 or 1536 floats at >= 1024 tokens with Anderson mixing of depth 3 or 4 at
    tolerance 0: the fused update and mix for wide rows (a lane's elements walked in groups, the
    rows in LDS) on the 256 x 256 tile paths.  (Depth 5 at these widths leaves up to 15% of the
    tokens ill-conditioned in the sense below.)"""
    rng = np.random.default_rng(5000 + seed)
    d = int(rng.choice([1024, 1536]))
    H = (2, 4)[seed % 2]
    V = int(rng.choice([600, 1500]))
    N = int(rng.choice([4, 16]))
    flags = synth.F_SCAN_SELECTIVE if rng.random() < 0.5 else 0
    for f in (synth.F_SCORE_CLAMP4, synth.F_RMS_EXCL_ANCHOR, synth.F_INIT_SIGNAL_RMS):
        if rng.random() < 0.3:
            flags |= f
    flags |= int(rng.choice([0, synth.F_RESID_L2]))
    m = int(rng.choice([3, 4]))
    B = int(rng.choice([1, 2]))
    T = int(rng.integers(1024, 1300)) // B
    mc = synth.ModelConfig(d=d, H=H, V=V, N=N, r=32, flags=flags, anderson_m=m, eps=0.0, max_iters=7,
                           qk_bias=bool(rng.random() < 0.3))
    return mc, B, T


@pytest.mark.parametrize("seed", range(4))
def test_random_wide_anderson_config_matches_oracle(oracle_lib, seed):
    mc, B, T = draw_wide(seed)
    log(f"random wide Anderson config {seed}: {mc} B={B} T={T}")
    w = synth.make_token_sensitive_weights(mc, seed=seed)
    toks = synth.make_tokens("zipf", B, T, mc.V, seed=seed)
    be = GpuDeqBackend(mc, B, T)
    be.upload_weights(w)
    got = be.forward(toks, want=ALL)
    be.close()
    check(oracle_lib, mc, w, toks, got, f"random wide Anderson config {seed}")
    assert (got["iters"] == mc.max_iters).all()


def draw_memory(seed):
    """The memory-coupled forward (fixed-history mode): position-sequential solves of B tokens
    with the history term, optional warm start, Anderson, and caller state."""
    rng = np.random.default_rng(3000 + seed)
    d = int(rng.choice([64, 128, 256]))
    H = int(rng.choice([1, 2, 4, 8]))
    V = int(rng.choice([300, 700]))
    flags = synth.F_MEMORY
    for f in (synth.F_SCORE_CLAMP4, synth.F_RMS_EXCL_ANCHOR, synth.F_TOKEN_CARRY, synth.F_INIT_SIGNAL_RMS):
        if rng.random() < 0.3:
            flags |= f
    m = int(rng.choice([0, 0, 2, 3]))
    eps = 0.0 if (m > 0 or rng.random() < 0.5) else 1e-4
    max_iters = int(rng.choice([3, 8, 12])) if eps == 0.0 else 20
    mc = synth.ModelConfig(d=d, H=H, V=V, N=1, r=32, flags=flags, anderson_m=m, eps=eps, max_iters=max_iters,
                           qk_bias=bool(rng.random() < 0.3))
    B, T = int(rng.integers(1, 5)), int(rng.integers(1, 14))
    return mc, B, T, bool(rng.random() < 0.5), bool(rng.random() < 0.5)


@pytest.mark.parametrize("seed", range(10))
def test_random_memory_config_matches_oracle(oracle_lib, seed):
    mc, B, T, strong, state_in = draw_memory(seed)
    log(f"random memory config {seed}: {mc} B={B} T={T} strong={strong} state_in={state_in}")
    w = dict(synth.make_token_sensitive_weights(mc, seed=seed))
    w.update(synth.make_hist_weights(mc, seed=seed + 1, strong=strong))
    toks = synth.make_tokens("uniform", B, T, mc.V, seed=seed)
    m_in = (0.5 * np.random.default_rng(seed).standard_normal((B, mc.H, mc.d))).astype(np.float32) if state_in else None
    be = GpuDeqBackend(mc, B, T)
    be.upload_weights(w)
    got = be.forward(toks, scan_state_in=None if m_in is None else m_in[..., None])
    be.close()
    ref = oracle_lib.Oracle(mc, w).forward_memory(toks, m_in=m_in, nthreads=16)
    ctx = f"random memory config {seed}"
    assert np.abs(got["iters"].astype(int) - ref["iters"].astype(int)).max() <= 1, ctx
    for g, r in (("h_star", "h_star"), ("pooled", "pooled"), ("logits", "logits"), ("scan_y", "m_seq")):
        np.testing.assert_allclose(got[g], ref[r], rtol=1e-4, atol=1e-3, err_msg=f"{ctx}: {g}")
    np.testing.assert_allclose(got["scan_state"][..., 0], ref["m_seq"][:, -1], rtol=1e-4, atol=1e-3,
                               err_msg=f"{ctx}: scan_state")
    bad = np.argwhere(got["argmax"] != ref["argmax"])
    for idx in bad:
        lg = np.sort(ref["logits"][tuple(idx)])
        assert lg[-1] - lg[-2] < 1e-5, f"{ctx}: argmax differs at {idx} without a near-tie"


def draw_decode(seed):
    """Greedy decode (Trainer::generate's loop, trainer.rs:4388-4406; the fixed-history form with
    ADN_F_MEMORY, :4395-4400): width, slots, flags, GEMM arithmetic, batch, prompt, window,
    generated count, Picard steps and repetition penalty."""
    rng = np.random.default_rng(4000 + seed)
    d = int(rng.choice([64, 128, 192, 256]))
    H = int(rng.choice([1, 2, 3, 4, 8]))
    V = int(rng.choice([300, 600]))
    flags = 0
    for f in (synth.F_SCORE_CLAMP4, synth.F_RMS_EXCL_ANCHOR, synth.F_INIT_SIGNAL_RMS, synth.F_WIN_TRANSPOSED):
        if rng.random() < 0.3:
            flags |= f
    flags |= int(rng.choice([0, 0, synth.F_GEMM_BF16X3, synth.F_GEMM_FP32]))
    memory = rng.random() < 0.3
    if memory:
        flags |= synth.F_MEMORY
    iters = int(rng.choice([2, 5, 10]))
    mc = synth.ModelConfig(d=d, H=H, V=V, N=1, r=32, flags=flags, eps=0.0, max_iters=iters,
                           qk_bias=bool(rng.random() < 0.3))
    B, T0 = int(rng.integers(1, 6)), int(rng.integers(1, 13))
    n_new = int(rng.integers(3, 9))
    ctx = int(rng.integers(1, T0 + n_new + 1))
    pen = float(rng.choice([1.0, 1.3]))
    return mc, B, T0, n_new, ctx, pen


@pytest.mark.parametrize("seed", range(12))
def test_random_decode_config_matches_oracle(oracle_lib, seed):
    mc, B, T0, n_new, ctx, pen = draw_decode(seed)
    log(f"random decode config {seed}: {mc} B={B} T0={T0} n_new={n_new} ctx={ctx} pen={pen}")
    w = dict(synth.make_token_sensitive_weights(mc, seed=seed))
    if mc.flags & synth.F_MEMORY:
        w.update(synth.make_hist_weights(mc, seed=seed + 1, strong=True))
    prompt = synth.make_tokens("uniform", B, T0, mc.V, seed=seed)
    ref = oracle_lib.Oracle(mc, w).decode_greedy(prompt, n_new, ctx, pen)
    be = GpuDeqBackend(mc, B, T0 if mc.flags & synth.F_MEMORY else 1)
    be.upload_weights(w)
    got = be.decode_greedy(prompt, n_new, ctx, max_iters=mc.max_iters, repetition_penalty=pen)
    be.close()
    assert np.array_equal(got, ref), f"decode config {seed}: {np.argwhere(got != ref)[:4].tolist()}"


def test_random_call_sequence_on_one_context(oracle_lib):
    """One context serving a seeded random sequence of calls of different shapes and kinds
    (token and row inputs, tolerance 0 or 1e-4, iteration caps, few-token and multi-sequence
    batches, greedy decodes with and without a penalty): every result against the oracle, so
    that no call depends on what an earlier one left in the context's buffers (active lists and
    counts, range-guard bounds, the small iterate buffers, exit flags, arg-max partials of either
    width, staging)."""
    mc0 = synth.ModelConfig(d=128, H=4, V=700, N=4, r=32, flags=synth.F_SCAN_SELECTIVE | synth.F_SCORE_CLAMP4)
    w = synth.make_token_sensitive_weights(mc0, seed=21)
    be = GpuDeqBackend(mc0, 4, 300)
    be.upload_weights(w)
    rng = np.random.default_rng(21)
    for call in range(16):
        kind = rng.choice(["forward", "s_in", "decode"])
        iters = int(rng.choice([2, 6, 20]))
        eps = 1e-4 if iters == 20 else 0.0
        mc = dataclasses.replace(mc0, max_iters=iters, eps=eps)
        if kind == "decode":
            B, T0 = int(rng.integers(1, 5)), int(rng.integers(1, 10))
            pen = float(rng.choice([1.0, 1.3]))
            prompt = synth.make_tokens("uniform", B, T0, mc.V, seed=100 + call)
            log(f"call {call}: decode B={B} T0={T0} iters={iters} pen={pen}")
            got = be.decode_greedy(prompt, 5, 8, max_iters=iters, repetition_penalty=pen)
            ref = oracle_lib.Oracle(dataclasses.replace(mc0, max_iters=iters, eps=0.0), w).decode_greedy(prompt, 5, 8, pen)
            assert np.array_equal(got, ref), f"call {call}"
            continue
        B = int(rng.integers(1, 5))
        T = int(rng.choice([1, 2, int(rng.integers(3, 300))]))
        toks = synth.make_tokens("uniform", B, T, mc.V, seed=100 + call)
        log(f"call {call}: {kind} B={B} T={T} iters={iters} eps={eps}")
        if kind == "forward":
            got = be.forward(toks, max_iters=iters, eps=eps, want=ALL)
        else:
            got = be.forward(s_in=np.ascontiguousarray(w["embed"][toks]), max_iters=iters, eps=eps, want=ALL)
        check(oracle_lib, mc, w, toks, got, f"call {call}")
    be.close()


@pytest.mark.parametrize("seed", range(8))
def test_random_adjoint_config_matches_oracle(oracle_lib, seed):
    """The clean adjoint Picard (staged_adjoint_picard_clean.wgsl:143-337) with its source gradient
    at random widths (multiples of 64, powers of two or not), slot counts, token counts, step
    counts and damping, without Anderson mixing (with it the coefficients of a nearly singular
    Gram system are compared elsewhere); both sides read the GPU forward's h*.  Bar as in
    test_gpu_adjoint: |got - ref| <= 1e-4 |ref| + 2e-5 max(1, max |ref|)."""
    rng = np.random.default_rng(5000 + seed)
    d = int(rng.choice([64, 128, 192, 320, 512, 768]))
    H = int(rng.choice([1, 2, 3, 4, 8]))
    mc = synth.ModelConfig(d=d, H=H, V=300, N=1, r=32)
    w = dict(synth.make_weights(mc, seed=seed))
    w["norm_scale"] = (1.0 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    B, T = int(rng.integers(1, 4)), int(rng.choice([1, 3, int(rng.integers(10, 200))]))
    iters = int(rng.integers(0, 13))
    damping = float(rng.choice([0.3, 0.7, 1.0]))
    toks = synth.make_tokens("uniform", B, T, mc.V, seed=seed)
    dl = rng.standard_normal((B, T, d)).astype(np.float32)
    log(f"random adjoint {seed}: d={d} H={H} B={B} T={T} iters={iters} damping={damping}")
    be = GpuDeqBackend(mc, B, T)
    be.upload_weights(w)
    h = be.forward(toks, want=("h_star",))["h_star"]
    v, src = be.adjoint(dl, iters, damping=damping)
    be.close()
    o = oracle_lib.Oracle(mc, w)
    sig = np.stack([o.signal(w["embed"][t]) for t in toks.reshape(-1)])
    vr, sr = o.adjoint(sig, h.reshape(B * T, H, d), dl.reshape(B * T, d), iters, beta=damping)
    for got, ref, what in ((v, vr.reshape(B, T, H, d), "v"), (src, sr.reshape(B, T, d), "source gradient")):
        np.testing.assert_allclose(got, ref, rtol=1e-4, atol=2e-5 * max(1.0, float(np.abs(ref).max())),
                                   err_msg=f"random adjoint {seed}: {what}")
