"""The fp16-split GEMMs outside the fp16 range, on the HIP path vs the CPU oracle (needs an MI355X).

The default GEMM arithmetic carries each fp32 operand as fp16 halves, whose range ends at 65504.
These models put every GEMM's A operand far beyond it -- the iterate h (and so the slot mix), the
LM head's normalised pooled row, the carrier output y, memory mode's state -- and must still meet
the forward's bar, the library scaling those operands down by powers of two.

The canonical cases are the ordinary model scaled by g = 2^16: norm_scale = lm_g = g and W_q, W_k,
W_v divided by g.  Then c = W_o mix + W_in x + anchor is unchanged for an iterate g h, so the fixed
point is g times the ordinary one with the same (contractive) dynamics: |h| reaches g sqrt(d)
bounds, the logits are g times the ordinary ones, and with W_B, W_C multiplied by 200 the carrier
output is 4 10^4 times the ordinary one.  Outputs are compared after dividing by those factors, at
rtol 1e-4 / atol 1e-3, iterations within +-1 and arg-max identical.
"""
import dataclasses

import numpy as np
import pytest

from aideen_amd import synth
from aideen_amd.backend import GpuDeqBackend

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-4, 1e-3
G = 65536.0


def log(msg):
    print(msg, flush=True)


def scaled_model(flags, anderson_m=0, d=2048, H=2, V=300, N=4):
    mc = synth.ModelConfig(d=d, H=H, V=V, N=N, r=32, flags=flags, anderson_m=anderson_m, eps=1e-4 * G,
                           max_iters=30)
    w = dict(synth.make_weights(mc, seed=3))
    for k in ("w_q", "w_k", "w_v"):
        w[k] = (w[k] / np.float32(G)).astype(np.float32)
    w["norm_scale"] = np.full(d, G, np.float32)
    w["lm_g"] = np.full(d, G, np.float32)
    w["w_b"] = (w["w_b"] * np.float32(200)).astype(np.float32)
    w["w_c"] = (w["w_c"] * np.float32(200)).astype(np.float32)
    return mc, w


@pytest.mark.parametrize("flags,anderson_m", [
    (synth.F_SCAN_SELECTIVE, 0),
    (synth.F_SCAN_SELECTIVE | synth.F_RMS_EXCL_ANCHOR, 0),  # the update's output bound is looser here
    (synth.F_SCAN_SELECTIVE, 3),                             # a mixed iterate raises the bound itself
])
def test_operands_beyond_fp16_range(oracle_lib, flags, anderson_m):
    log(f"range guard flags={flags} anderson={anderson_m}")
    mc, w = scaled_model(flags, anderson_m)
    B, T = 2, 9
    toks = synth.make_tokens("uniform", B, T, mc.V, seed=4)
    be = GpuDeqBackend(mc, B, T)
    be.upload_weights(w)
    got = be.forward(toks)
    ref = oracle_lib.Oracle(mc, w).forward(toks, nthreads=16)
    assert np.abs(got["h_star"]).max() > 65504 and np.abs(got["scan_y"]).max() > 2 * 65504
    for k, v in got.items():
        if v.dtype.kind == "f":
            assert np.isfinite(v).all(), k
    assert np.abs(got["iters"].astype(int) - ref["iters"]).max() <= 1
    assert np.array_equal(got["converged"], ref["converged"])
    for k, f in (("h_star", G), ("pooled", G), ("logits", G), ("scan_y", 4e4), ("scan_state", 200.0)):
        np.testing.assert_allclose(got[k] / f, ref[k] / f, rtol=RTOL, atol=ATOL, err_msg=k)
    assert np.array_equal(got["argmax"], ref["argmax"])


def test_operands_beyond_fp16_range_wide_tiles(oracle_lib):
    """The same scaled model with 1024 tokens at d = 512, V = 600: W_o and the LM head run on the
    256x256 tiles, whose A operands (the slot mix, the normalised pooled row) their producers write
    already split into fp16 halves, at the scale the GEMM derives from the h bound (mix) or the
    head's static bound (pooled row)."""
    log("range guard on the 256x256 tiles: d=512 H=2 V=600, 1024 tokens")
    mc, w = scaled_model(synth.F_SCAN_SELECTIVE, 0, d=512, H=2, V=600)
    B, T = 4, 256
    toks = synth.make_tokens("uniform", B, T, mc.V, seed=6)
    be = GpuDeqBackend(mc, B, T)
    be.upload_weights(w)
    got = be.forward(toks)
    ref = oracle_lib.Oracle(mc, w).forward(toks, nthreads=16)
    assert np.abs(got["h_star"]).max() > 65504
    for k, v in got.items():
        if v.dtype.kind == "f":
            assert np.isfinite(v).all(), k
    assert np.abs(got["iters"].astype(int) - ref["iters"]).max() <= 1
    for k, f in (("h_star", G), ("pooled", G), ("logits", G), ("scan_y", 4e4), ("scan_state", 200.0)):
        np.testing.assert_allclose(got[k] / f, ref[k] / f, rtol=RTOL, atol=ATOL, err_msg=k)
    assert np.array_equal(got["argmax"], ref["argmax"])


def test_memory_state_beyond_fp16_range(oracle_lib):
    """Memory mode with a carried state of magnitude ~10^6: the W_hist product of m_{t-1} and the
    W_out readout of the carrier state run on operands beyond the fp16 range."""
    log("range guard, memory mode")
    mc = synth.ModelConfig(d=256, H=4, V=300, N=1, r=32, flags=synth.F_MEMORY)
    w = dict(synth.make_weights(mc, seed=3))
    w.update(synth.make_hist_weights(mc, seed=11, strong=True))
    B, T = 2, 6
    toks = synth.make_tokens("uniform", B, T, mc.V, seed=5)
    m_in = synth.uniform(9, "m_in", (B, mc.H, mc.d, 1), -1e6, 1e6)
    be = GpuDeqBackend(mc, B, T)
    be.upload_weights(w)
    got = be.forward(toks, scan_state_in=m_in)
    ref = oracle_lib.Oracle(mc, w).forward_memory(toks, m_in=m_in[..., 0])
    assert np.abs(got["scan_y"][:, 0]).max() > 65504
    assert np.abs(got["iters"].astype(int) - ref["iters"]).max() <= 1
    for k in ("h_star", "pooled", "logits"):
        np.testing.assert_allclose(got[k], ref[k], rtol=RTOL, atol=ATOL, err_msg=k)
    np.testing.assert_allclose(got["scan_y"], ref["m_seq"], rtol=RTOL, atol=ATOL + 1e-7 * 1e6, err_msg="m_seq")
    assert np.array_equal(got["argmax"], ref["argmax"])
