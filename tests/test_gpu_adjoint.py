"""The clean adjoint Picard (the reference's backward for the solve; staged_adjoint_picard_clean.wgsl:
143-337, gpu_deq.rs:4736-4975) on the HIP path vs the oracle's restatement, through the C ABI
(needs an MI355X).  Both read the same h* (the GPU forward's); the signal is each side's own
W_in x.  Bar: |got - ref| <= 1e-4 |ref| + 2e-5 max(1, max |ref|) on v and on the source gradient
(the absolute part scales with the largest entry: the adjoint iteration can amplify its
right-hand side by orders of magnitude, and rounding grows with it).  With Anderson mixing the
absolute part is 1e-3 (the forward's bar): the mixing coefficients solve a nearly singular Gram
system of differences of close iterates, which magnifies the two sides' rounding differences."""
import dataclasses

import numpy as np
import pytest
# torch (device buffers for the async form) brings its own HIP runtime: imported before the
# library is first loaded so that one runtime serves both
import torch

from aideen_amd import synth
from aideen_amd._lib import AdnError
from aideen_amd.backend import GpuDeqBackend

pytestmark = pytest.mark.gpu
RTOL, ATOL = 1e-4, 2e-5


def close(got, ref, what, atol=ATOL):
    np.testing.assert_allclose(got, ref, rtol=RTOL, atol=atol * max(1.0, float(np.abs(ref).max())), err_msg=what)


def log(msg):
    print(msg, flush=True)


def setup(d, H, V=300, anderson_m=0, B=2, T=9, seed=4):
    mc = synth.ModelConfig(d=d, H=H, V=V, N=1, r=32, flags=0, anderson_m=anderson_m)
    w = dict(synth.make_weights(mc, seed=seed))
    rng = np.random.default_rng(seed)
    w["norm_scale"] = (1.0 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    toks = synth.make_tokens("uniform", B, T, V, seed=seed + 1)
    dl = rng.standard_normal((B, T, d)).astype(np.float32)
    return mc, w, toks, dl


def oracle_adjoint(oracle_lib, mc, w, toks, h_star, dl, iters):
    o = oracle_lib.Oracle(mc, w)
    B, T = toks.shape
    sig = np.stack([o.signal(w["embed"][t]) for t in toks.reshape(-1)])
    v, src = o.adjoint(sig, h_star.reshape(B * T, mc.H, mc.d), dl.reshape(B * T, mc.d), iters)
    return v.reshape(B, T, mc.H, mc.d), src.reshape(B, T, mc.d)


CASES = [
    dict(d=64, H=1, iters=0), dict(d=64, H=4, iters=1), dict(d=128, H=4, iters=2),
    dict(d=128, H=8, iters=10), dict(d=512, H=8, iters=2), dict(d=256, H=2, iters=40),
    dict(d=128, H=4, iters=6, anderson_m=3), dict(d=128, H=8, iters=3, anderson_m=4),
    # widths other than powers of two (the reference's benchmark width 192) and odd slot counts
    dict(d=192, H=6, iters=2), dict(d=320, H=3, iters=0), dict(d=1536, H=5, iters=3),
]
# With three or more residuals (anderson_m >= 4 past the third step) the mixing solves a 3x3 (4x4)
# Gram system of differences of the adjoint's nearly collinear iterates: condition numbers 4e5-2e6
# before the 1e-4 trace regularisation (about 1e4 after), so the coefficients of two summation
# orders differ by percents and an element-wise comparison is meaningless there.  Those steps are
# pinned in the oracle step by step (test_adjoint_anderson_bookkeeping); here m = 4 is compared
# through its first mix (ring slot k % 4).


@pytest.mark.parametrize("case", CASES, ids=lambda c: "-".join(f"{k}{c[k]}" for k in c))
def test_adjoint_matches_oracle(oracle_lib, case):
    log(f"adjoint {case}")
    mc, w, toks, dl = setup(case["d"], case["H"], anderson_m=case.get("anderson_m", 0))
    be = GpuDeqBackend(mc, *toks.shape)
    be.upload_weights(w)
    h = be.forward(toks, want=("h_star",))["h_star"]
    v, src = be.adjoint(dl, case["iters"])
    vr, sr = oracle_adjoint(oracle_lib, mc, w, toks, h, dl, case["iters"])
    atol = 1e-3 if case.get("anderson_m", 0) else ATOL
    close(v, vr, "v", atol)
    close(src, sr, "source gradient", atol)


def test_adjoint_fixed_point_and_explicit_h(oracle_lib):
    """Enough steps reach the adjoint fixed point: one more step changes nothing beyond rounding;
    an explicit h* equal to the forward's gives the same result.  The iteration contracts only
    when the signal dominates pre = signal + h*: h* is an RMSNorm output scaled by g, so with a
    small signal |g| / rms(pre) ~ 1 and the step's spectral radius is ~ beta + (1 - beta) = 1 (the
    reference runs two steps and does not need convergence).  Large s_in rows make it contract."""
    log("adjoint fixed point")
    mc, w, toks, dl = setup(512, 8, V=1000, B=4, T=33)
    be = GpuDeqBackend(mc, *toks.shape)
    be.upload_weights(w)
    s_in = (10.0 * np.random.default_rng(9).standard_normal(toks.shape + (mc.d,))).astype(np.float32)
    h = be.forward(s_in=s_in, want=("h_star",))["h_star"]
    v60, _ = be.adjoint(dl, 60)
    v61, _ = be.adjoint(dl, 61)
    assert np.abs(v61 - v60).max() < 1e-5 * max(1.0, np.abs(v60).max())
    v2, s2 = be.adjoint(dl, 3)
    v3, s3 = be.adjoint(dl, 3, h_star=h)
    assert np.array_equal(v2, v3) and np.array_equal(s2, s3)


def test_adjoint_async_equals_blocking():
    log("adjoint async")
    mc, w, toks, dl = setup(256, 4)
    B, T = toks.shape
    be = GpuDeqBackend(mc, B, T)
    be.upload_weights(w)
    be.forward(toks, want=("h_star",))
    v, src = be.adjoint(dl, 4)
    dev = torch.device("cuda:0")
    vd = torch.empty((B, T, mc.H, mc.d), device=dev)
    sd = torch.empty((B, T, mc.d), device=dev)
    be.adjoint_async(B * T, torch.from_numpy(dl).to(dev), 4, mc.beta, vd, sd)
    be.synchronize()
    assert np.array_equal(vd.cpu().numpy(), v) and np.array_equal(sd.cpu().numpy(), src)


def test_adjoint_errors():
    log("adjoint errors")
    mc, w, toks, dl = setup(64, 2)
    be = GpuDeqBackend(mc, *toks.shape)
    be.upload_weights(w)
    with pytest.raises(AdnError, match="before a forward"):
        be.adjoint(dl, 2)
    be.forward(toks, want=("h_star",))
    with pytest.raises(AdnError, match="token count"):
        be.adjoint(dl[:1], 2)
    with pytest.raises(AdnError, match="iters"):
        be.adjoint(dl, -1)
    with pytest.raises(AdnError, match="damping"):
        be.adjoint(dl, 2, damping=0.0)
