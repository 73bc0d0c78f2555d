"""Forward parity that can fail on a per-token error (needs an MI355X).

With the reference's own initialisation (anchors U(-1, 1), fixed_point_memory_reasoning.rs:225-232;
the golden-ratio closed forms of E and W_lm, tokenizer.rs:62-66, lm_head.rs:24-29) the solve is
anchor-dominated: at the north-star shape every token's arg-max is the same and the logits'
token-dependent part is below the forward's atol, so a logits row written to the wrong token
would pass a tolerance check.  These tests run synth.make_token_sensitive_weights, where the
signal dominates, and each asserts first that its comparison can fail (as the reference's
pipeline test asserts of its own, picard_pipeline_test.rs:1021-1030): the oracle's arg-max takes
at least 16 distinct values and the logits' token-dependent spread is at least 10x atol.

The LM head is lm_head.rs:50-54 (RMSNorm of the slot mean, W_lm, bias) with the last-max arg-max
of lm_head.rs:62-69; greedy decode is trainer.rs:4388-4406.
"""
import dataclasses

import numpy as np
import pytest

from aideen_amd import synth
from aideen_amd.backend import GpuDeqBackend
from test_gpu_parity import ATOL, RTOL, assert_forward_parity, last_max, log

pytestmark = pytest.mark.gpu

ALL = ("h_star", "pooled", "logits", "argmax", "iters", "converged", "scan_y", "scan_state")


def assert_discriminating(ref, ctx):
    """The oracle's outputs on these tokens differ from token to token by far more than the bar."""
    am = ref["argmax"].ravel()
    lg = ref["logits"].reshape(-1, ref["logits"].shape[-1])
    spread = float(np.abs(lg - lg.mean(axis=0)).max())
    log(f"{ctx}: {len(set(am.tolist()))} distinct arg-max values over {am.size} tokens, logit spread {spread:.3f}")
    assert len(set(am.tolist())) >= 16, f"{ctx}: arg-max takes too few values to discriminate tokens"
    assert spread >= 10 * ATOL, f"{ctx}: logits' token-dependent part {spread:.2e} is below 10x atol"


def assert_shift_fails(got_rows, ref_rows, tok_rows, ctx):
    """A one-row shift of the GPU rows against the oracle's (row i compared with row i+1) is
    outside the bar wherever the two rows hold different token ids, so a row-mapping error cannot
    pass."""
    g, r = got_rows[:-1], ref_rows[1:]
    differ = np.asarray(tok_rows[:-1]) != np.asarray(tok_rows[1:])
    outside = (np.abs(g - r) > ATOL + RTOL * np.abs(r)).reshape(g.shape[0], -1).any(axis=1)
    assert differ.sum() >= 8, f"{ctx}: too few neighbouring rows with different tokens"
    assert outside[differ].all(), f"{ctx}: a one-row shift would pass on {(~outside[differ]).sum()} rows"


def test_ns_token_sensitive_sampled_parity():
    """North-star shape (B=32, T=256, d=512, H=8, V=50257, N=16) on the token-sensitive weights.
    One token in each of the LM head's 32 persistent 256-row tiles (one sequence each), at a
    different row of the tile every time, plus both ends of two sequences: h*, pooled, iterations,
    converged and the full 50,257-wide logits rows and arg-max against the oracle.  The carrier
    output and final state of two whole sequences against the oracle's scan of the GPU's h*; over
    all 8192 tokens the fused arg-max equals the last-max of the stored logits."""
    from oracle import pyoracle
    p = synth.PRESETS["NS"]
    mc = p["model"]
    B, T = p["B"], p["T"]
    w = synth.make_token_sensitive_weights(mc)
    toks = synth.make_tokens(p["tokens"], B, T, mc.V, seed=1)
    be = GpuDeqBackend(mc, B, T)
    be.upload_weights(w)
    log("NS token-sensitive forward")
    got = be.forward(toks, want=ALL)
    be.close()
    assert got["converged"].all() and got["iters"].max() < mc.max_iters
    idx = [(j, (37 * j + 5) % T) for j in range(B)] + [(0, 0), (0, T - 1), (B - 1, 0), (B - 1, T - 1)]
    o = pyoracle.Oracle(mc, w)
    sub = np.array([[toks[b, t] for b, t in idx]], np.int32)
    ref = o.forward(sub, want_scan=False, nthreads=16)
    assert_discriminating(ref, "NS sample")
    keys = ("h_star", "pooled", "logits", "argmax", "iters", "converged")
    gsub = {k: np.stack([got[k][b, t] for b, t in idx])[None] for k in keys}
    assert_forward_parity(gsub, ref, "NS token-sensitive sample")
    assert np.array_equal(gsub["argmax"], ref["argmax"])
    assert_shift_fails(gsub["logits"][0], ref["logits"][0], sub[0], "NS logits")
    assert_shift_fails(gsub["h_star"][0], ref["h_star"][0], sub[0], "NS h*")
    assert len(set(got["iters"].ravel().tolist())) >= 2  # iteration counts vary over the batch
    for b in (0, B - 1):
        log(f"NS token-sensitive scan of sequence {b}")
        y, st = o.scan(got["h_star"][b])
        np.testing.assert_allclose(got["scan_y"][b], y, rtol=RTOL, atol=ATOL, err_msg=f"scan_y[{b}]")
        np.testing.assert_allclose(got["scan_state"][b], st, rtol=RTOL, atol=ATOL, err_msg=f"scan_state[{b}]")
    np.testing.assert_allclose(got["pooled"], got["h_star"].mean(axis=2), rtol=1e-5, atol=1e-6)
    for b in range(B):
        assert np.array_equal(got["argmax"][b], last_max(got["logits"][b])), f"arg-max vs logits, seq {b}"


@pytest.mark.parametrize("kind", ["preset", "token_sensitive"])
def test_ns_position_permutation_is_bit_exact(kind):
    """Every token's solve, pooling, logits row and arg-max depend on that token alone: permuting
    the 8192 positions of the north-star batch permutes the h*, logits and arg-max rows bit for
    bit (the GEMM tiles, the active-list order and the LM head's 256-row tiles all change).  With
    the reference's initialisation this catches row-mapping errors that a tolerance check on its
    near-identical logits rows would not."""
    p = synth.PRESETS["NS"]
    mc = p["model"]
    B, T = p["B"], p["T"]
    w = synth.weights_of_kind(kind, mc)
    toks = synth.make_tokens(p["tokens"], B, T, mc.V, seed=1)
    perm = np.random.default_rng(3).permutation(B * T)
    toks2 = toks.reshape(-1)[perm].reshape(B, T)
    be = GpuDeqBackend(mc, B, T)
    be.upload_weights(w)
    want = ("h_star", "logits", "argmax", "iters")
    log(f"NS permutation ({kind}): forward 1")
    a = be.forward(toks, want=want)
    log(f"NS permutation ({kind}): forward 2")
    b = be.forward(toks2, want=want)
    be.close()
    for k in want:
        ra = a[k].reshape((B * T,) + a[k].shape[2:])
        rb = b[k].reshape((B * T,) + b[k].shape[2:])
        assert np.array_equal(rb, ra[perm]), f"{kind}: {k} rows do not permute bit for bit"


# at least 1024 tokens with V >= 512: the persistent 256x256 tiles of every GEMM role and the LM
# head's arg-max epilogue, a time-chunked carrier; every output of every token
LARGE_TS = [
    dict(d=128, H=4, V=4096, N=16, flags=synth.F_SCAN_SELECTIVE, B=4, T=512),
    dict(d=512, H=2, V=2048, N=4, flags=synth.F_SCAN_SELECTIVE | synth.F_SCORE_CLAMP4, qk_bias=True, B=2, T=640),
]


@pytest.mark.parametrize("var", LARGE_TS, ids=lambda v: "-".join(f"{k}{v[k]}" for k in v))
def test_large_token_sensitive_every_output(oracle_lib, var):
    var = dict(var)
    B, T = var.pop("B"), var.pop("T")
    log(f"large token-sensitive {var} B={B} T={T}")
    mc = synth.ModelConfig(r=32, **var)
    w = synth.make_token_sensitive_weights(mc, seed=3)
    toks = synth.make_tokens("zipf", B, T, mc.V, seed=9)
    be = GpuDeqBackend(mc, B, T)
    be.upload_weights(w)
    got = be.forward(toks, want=ALL)
    be.close()
    ref = oracle_lib.Oracle(mc, w).forward(toks, nthreads=16)
    assert_discriminating(ref, f"large {var}")
    assert_forward_parity(got, ref, f"large token-sensitive {var}")
    assert np.array_equal(got["argmax"], ref["argmax"])
    for b in range(B):
        assert_shift_fails(got["logits"][b], ref["logits"][b], toks[b], f"logits seq {b}")
    assert np.array_equal(got["argmax"], last_max(got["logits"]))


@pytest.mark.parametrize("pen", [1.0, 1.3])
def test_c2_token_sensitive_forward_and_decode(oracle_lib, pen):
    """C2 (d=512, H=8, V=50257, N=16, B=1, T=256) on the token-sensitive weights: every output of
    every position against the oracle, then the 64-token greedy decode from the 256 tokens (ctx_len
    256, generate's 10 Picard steps) token for token, without and with a repetition penalty
    (lm_head.rs:81-99).  The decoded tokens vary (a decode that repeats one token would pass on any
    error that keeps it)."""
    p = synth.PRESETS["C2"]
    mc = p["model"]
    w = synth.make_token_sensitive_weights(mc)
    toks = synth.make_tokens(p["tokens"], p["B"], p["T"], mc.V, seed=1)
    be = GpuDeqBackend(mc, p["B"], p["T"])
    be.upload_weights(w)
    if pen == 1.0:
        log("C2 token-sensitive forward")
        got = be.forward(toks, want=ALL)
        ref = oracle_lib.Oracle(mc, w).forward(toks, nthreads=16)
        assert_discriminating(ref, "C2")
        assert_forward_parity(got, ref, "C2 token-sensitive")
        assert np.array_equal(got["argmax"], ref["argmax"])
        assert_shift_fails(got["logits"][0], ref["logits"][0], toks[0], "C2 logits")
    log(f"C2 token-sensitive decode pen={pen}")
    mcd = dataclasses.replace(mc, max_iters=10, eps=0.0)
    dref = oracle_lib.Oracle(mcd, w).decode_greedy(toks, 64, 256, pen)
    distinct = len(set(dref.ravel().tolist()))
    log(f"C2 decode pen={pen}: {distinct} distinct tokens, {int((dref[0, 1:] != dref[0, :-1]).sum())} changes")
    assert distinct >= (16 if pen != 1.0 else 8)
    dec = be.decode_greedy(toks, 64, 256, repetition_penalty=pen)
    be.close()
    assert np.array_equal(dec, dref), np.flatnonzero(dec[0] != dref[0])[:5]
