"""Memory-coupled forward (ADN_F_MEMORY) on the HIP path vs the CPU oracle, through the C ABI.

The reference's fixed-history mode (trainer.rs:677-720): each token's Picard solve adds the
history context of the carrier state m_{t-1} (fixed_point_memory_reasoning.rs:1317-1370) and
m_t = temporal_step(m_{t-1}, h*_t) (fixed_point_memory_reasoning.rs:1454-1485).  Bar as for the
canonical forward: rtol 1e-4 / atol 1e-3 on h*, pooled, logits and every carrier state m_t,
iteration counts within +-1, arg-max identical except at genuine near-ties.
"""
import dataclasses

import numpy as np
import pytest
# torch (device buffers for the profiled forward) brings its own HIP runtime: it is imported
# before the library is first loaded so that one runtime serves both
import torch

from aideen_amd import synth
from aideen_amd._lib import AdnError
from aideen_amd.backend import GpuDeqBackend

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-4, 1e-3


def log(msg):
    print(msg, flush=True)


def mem_model(d, H, V, strong=True, w_out=True, **kw):
    kw.setdefault("flags", 0)
    kw["flags"] |= synth.F_MEMORY
    mc = synth.ModelConfig(d=d, H=H, V=V, N=1, r=32, **kw)
    w = dict(synth.make_weights(mc, seed=3))
    w.update(synth.make_hist_weights(mc, seed=11, strong=strong))
    if not w_out:
        w["w_out"] = None
    return mc, w


def gpu_memory(mc, w, toks, m_in=None, B=None, T=None):
    B0, T0 = toks.shape
    be = GpuDeqBackend(mc, B or B0, T or T0)
    be.upload_weights(w)
    return be.forward(toks, scan_state_in=m_in)


def check(got, ref, ctx):
    di = np.abs(got["iters"].astype(int) - ref["iters"].astype(int))
    assert di.max() <= 1, f"{ctx}: iteration counts differ by {di.max()}"
    pairs = [("h_star", "h_star"), ("pooled", "pooled"), ("logits", "logits"), ("scan_y", "m_seq")]
    for g, r in pairs:
        np.testing.assert_allclose(got[g], ref[r], rtol=RTOL, atol=ATOL, err_msg=f"{ctx}: {g}")
    np.testing.assert_allclose(got["scan_state"][..., 0], ref["m_seq"][:, -1], rtol=RTOL, atol=ATOL,
                               err_msg=f"{ctx}: scan_state")
    bad = np.argwhere(got["argmax"] != ref["argmax"])
    for idx in bad:
        lg = np.sort(ref["logits"][tuple(idx)])
        assert lg[-1] - lg[-2] < 1e-5, f"{ctx}: argmax differs at {idx} without a near-tie"
    assert len(bad) <= max(1, ref["argmax"].size // 100)


MEM_VARIANTS = [
    dict(d=64, H=1, V=300),
    dict(d=128, H=4, V=500, eps=0.0, max_iters=12),  # fixed iteration count, as the reference runs it
    dict(d=128, H=4, V=500, w_out=False),
    dict(d=128, H=8, V=1000, qk_bias=True, flags=synth.F_SCORE_CLAMP4),
    dict(d=256, H=4, V=700, strong=False),  # the reference's initial history weights
    dict(d=128, H=4, V=500, sigma=0.7, anderson_m=3),
    dict(d=128, H=4, V=500, flags=synth.F_TOKEN_CARRY),  # warm start from h*_{t-1}
    dict(d=256, H=8, V=700, flags=synth.F_TOKEN_CARRY | synth.F_INIT_SIGNAL_RMS, anderson_m=2),
    # the fused update-and-mix kernel for wide rows with the history term (1024, and 1536: not a
    # power of two), at tolerance 0 so that every position runs all 8 steps
    dict(d=1024, H=2, V=400, sigma=0.7, anderson_m=3, eps=0.0, max_iters=8),
    dict(d=1536, H=2, V=400, sigma=0.7, anderson_m=3, eps=0.0, max_iters=8),
]


@pytest.mark.parametrize("var", MEM_VARIANTS, ids=lambda v: "-".join(f"{k}{v[k]}" for k in v))
def test_memory_forward_matches_oracle(oracle_lib, var):
    log(f"memory variant {var}")
    mc, w = mem_model(**var)
    B, T = 3, 13  # ragged
    toks = synth.make_tokens("uniform", B, T, mc.V, seed=5)
    ref = oracle_lib.Oracle(mc, w).forward_memory(toks)
    got = gpu_memory(mc, w, toks)
    check(got, ref, str(var))
    if mc.eps == 0.0:
        assert np.all(got["iters"] == mc.max_iters)


def test_memory_state_in_and_continuation(oracle_lib):
    """A caller-supplied m_{-1} is the history of the first token, and running a sequence in
    two pieces with the carrier state passed across equals the whole run."""
    log("memory continuation")
    mc, w = mem_model(128, 4, 500, eps=0.0, max_iters=10)
    toks = synth.make_tokens("uniform", 2, 11, mc.V, seed=7)
    o = oracle_lib.Oracle(mc, w)
    m_in = (0.5 * np.random.default_rng(4).standard_normal((2, mc.H, mc.d))).astype(np.float32)
    ref = o.forward_memory(toks, m_in=m_in)
    be = GpuDeqBackend(mc, 2, 11)
    be.upload_weights(w)
    got = be.forward(toks, scan_state_in=m_in[..., None])
    check(got, ref, "state in")
    a = be.forward(toks[:, :5])
    b = be.forward(toks[:, 5:], scan_state_in=a["scan_state"])
    full = be.forward(toks)
    for k in ("h_star", "scan_y", "logits"):
        np.testing.assert_allclose(np.concatenate([a[k], b[k]], axis=1), full[k], rtol=1e-5, atol=1e-5,
                                   err_msg=k)
    np.testing.assert_allclose(b["scan_state"], full["scan_state"], rtol=1e-5, atol=1e-5)


def test_memory_first_token_is_the_canonical_solve():
    """Without a carrier state the first token has no history: its h* equals the canonical
    forward's (same weights, memory flag off)."""
    log("memory first token")
    mc, w = mem_model(128, 4, 500)
    toks = synth.make_tokens("uniform", 4, 6, mc.V, seed=8)
    got = gpu_memory(mc, w, toks)
    canon_mc = dataclasses.replace(mc, flags=mc.flags & ~synth.F_MEMORY)
    be = GpuDeqBackend(canon_mc, 4, 6)
    be.upload_weights(w)
    canon = be.forward(toks, want=("h_star", "iters"))
    np.testing.assert_allclose(got["h_star"][:, 0], canon["h_star"][:, 0], rtol=1e-5, atol=1e-5)
    assert np.array_equal(got["iters"][:, 0], canon["iters"][:, 0])
    assert np.abs(got["h_star"][:, 1:] - canon["h_star"][:, 1:]).max() > 1e-3


def test_memory_s_in_path_equals_token_path():
    log("memory s_in")
    mc, w = mem_model(128, 4, 500)
    toks = synth.make_tokens("uniform", 2, 7, mc.V, seed=9)
    be = GpuDeqBackend(mc, 2, 7)
    be.upload_weights(w)
    a = be.forward(toks)
    b = be.forward(s_in=w["embed"][toks])
    for k in ("h_star", "scan_y", "logits"):
        np.testing.assert_allclose(a[k], b[k], rtol=1e-6, atol=1e-6, err_msg=k)


def test_memory_errors():
    log("memory errors")
    mc, w = mem_model(64, 2, 100)
    be = GpuDeqBackend(mc, 2, 4)
    w_missing = dict(w)
    w_missing["w_hist"] = None
    with pytest.raises(AdnError, match="w_hist"):
        be.upload_weights(w_missing)
    be.upload_weights(w)
    mcc, wc = mem_model(64, 2, 100, flags=synth.F_TOKEN_CARRY)
    bc = GpuDeqBackend(mcc, 2, 4)
    bc.upload_weights(wc)
    with pytest.raises(AdnError, match="TOKEN_CARRY"):
        bc.decode_greedy(np.array([[1, 2], [3, 4]], np.int32), 3, 4)


def test_memory_reference_shape(oracle_lib):
    """A width and slot count other than powers of two (d = 192, H = 6) in memory mode."""
    log("memory d=192 H=6")
    mc, w = mem_model(192, 6, 300)
    toks = synth.make_tokens("uniform", 2, 11, mc.V, seed=15)
    check(gpu_memory(mc, w, toks), oracle_lib.Oracle(mc, w).forward_memory(toks), "d192 H6")


@pytest.mark.parametrize("pen", [1.0, 1.5])
def test_memory_greedy_decode_matches_oracle(oracle_lib, pen):
    """The fixed-history form of Trainer::generate (trainer.rs:4395-4400, 677-735): the memory is
    primed over the prompt, then each step solves the last token with the memory's history
    context (eps = 0: the reference's fixed max_iters) and advances the memory."""
    log(f"memory decode pen={pen}")
    mc, w = mem_model(128, 4, 400, max_iters=6, eps=0.0)
    prompt = synth.make_tokens("uniform", 3, 7, mc.V, seed=14)
    ref = oracle_lib.Oracle(mc, w).decode_greedy(prompt, 9, 5, pen)
    be = GpuDeqBackend(mc, 3, 7)
    be.upload_weights(w)
    got = be.decode_greedy(prompt, 9, 5, max_iters=6, eps=0.0, repetition_penalty=pen)
    assert np.array_equal(got, ref)


def test_memory_profile_counts():
    """adn_profile_forward in memory mode: the active tokens per iteration, summed over the
    positions, add up to every token's iteration count; one launch per position and iteration."""
    log("memory profile")
    mc, w = mem_model(128, 4, 500)
    B, T = 3, 9
    toks = synth.make_tokens("uniform", B, T, mc.V, seed=12)
    be = GpuDeqBackend(mc, B, T)
    be.upload_weights(w)
    dev = torch.device("cuda:0")
    outs = dict(h_star=torch.empty((B, T, mc.H, mc.d), device=dev),
                iters=torch.empty((B, T), dtype=torch.int32, device=dev),
                logits=torch.empty((B, T, mc.V), device=dev),
                argmax=torch.empty((B, T), dtype=torch.int32, device=dev),
                scan_y=torch.empty((B, T, mc.H, mc.d), device=dev),
                scan_state=torch.empty((B, mc.H, mc.d, 1), device=dev))
    prof = be.profile_forward(torch.from_numpy(toks).to(dev), outputs=outs)
    iters = outs["iters"].cpu().numpy()
    assert sum(prof["active"]) == int(iters.sum())
    assert prof["active"][0] == B * T
    st = prof["stages"]
    assert st["qkv_gemm"]["launches"] == T * mc.max_iters
    assert st["temporal"]["launches"] == T and st["hist_gemm"]["launches"] == T - 1
    ref = be.forward(toks)
    np.testing.assert_array_equal(outs["argmax"].cpu().numpy(), ref["argmax"])


def test_token_carry_repeated_token_converges_at_once():
    """With zero history and the same token at every position, a warm-started solve begins at
    its own fixed point: one iteration per position after the first, as the oracle pins."""
    log("token carry repeated token")
    mc, w = mem_model(128, 4, 500, flags=synth.F_TOKEN_CARRY, eps=1e-5, max_iters=40)
    w["w_hist"] = np.zeros_like(w["w_hist"])
    w["hist_slot_scale"] = np.zeros_like(w["hist_slot_scale"])
    toks = np.full((2, 6), 17, np.int32)
    got = gpu_memory(mc, w, toks)
    assert got["iters"][0, 0] > 3
    assert np.all(got["iters"][:, 1:] == 1)


def test_memory_batch_beyond_max_batch(oracle_lib):
    """A context created with max_batch = 1, max_seq = 8 (an .aidn-derived shape) admits any
    batch * seq <= 8: a memory forward at batch 2 x seq 4, and a fixed-history decode of batch 2
    whose priming runs 2 x 4 prompt tokens, both against the oracle.  Every per-position buffer of
    the memory driver ([batch][H][d]) must hold that batch."""
    log("memory batch beyond max_batch")
    mc, w = mem_model(128, 4, 400, max_iters=6, eps=0.0)
    toks = synth.make_tokens("uniform", 2, 4, mc.V, seed=16)
    be = GpuDeqBackend(mc, 1, 8)
    be.upload_weights(w)
    o = oracle_lib.Oracle(mc, w)
    check(be.forward(toks), o.forward_memory(toks), "batch 2 x seq 4 on max_batch 1")
    got = be.decode_greedy(toks, 3, 4, max_iters=6, eps=0.0)
    assert np.array_equal(got, o.decode_greedy(toks, 3, 4, 1.0))
    with pytest.raises(AdnError, match="capacity"):
        be.forward(synth.make_tokens("uniform", 3, 3, mc.V, seed=17))
