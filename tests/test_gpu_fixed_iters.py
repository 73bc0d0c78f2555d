"""Few-token solves with a fixed iteration count (needs an MI355X).

With at most four tokens, a tolerance of zero (no token can exit before the last iteration), no
plateau exit, no Anderson mixing and no history term, each Q|K|V product applies the previous
iteration's damped update itself (fixed_point_memory_reasoning.rs:1386-1393) and the update
kernel runs only at the last iteration, where it records the iteration counts.  A tolerance of
1e-30 exits no token either (every residual here stays far above it) but runs the update kernel
at every iteration: the two runs must agree bit for bit, and match the oracle.  A greedy decode
(generate's 10 steps at tolerance 0) takes the first form at every step.
"""
import dataclasses

import numpy as np
import pytest

from aideen_amd import synth
from aideen_amd.backend import GpuDeqBackend
from test_gpu_parity import assert_forward_parity, log

pytestmark = pytest.mark.gpu

ALL = ("h_star", "pooled", "logits", "argmax", "iters", "converged")

CASES = [
    # d = 512, H = 8: four waves per Q|K|V block, one row each
    dict(d=512, H=8, V=3000, N=4, flags=synth.F_SCAN_SELECTIVE, B=1, T=4),
    dict(d=512, H=8, V=3000, N=4, flags=synth.F_SCAN_SELECTIVE, B=1, T=1),
    # d = 128: two waves per block, two rows each; the anchor left out of the RMS, q/k bias
    dict(d=128, H=4, V=500, N=2, flags=synth.F_RMS_EXCL_ANCHOR | synth.F_SCORE_CLAMP4, qk_bias=True, B=2, T=2),
    dict(d=128, H=4, V=500, N=2, flags=synth.F_INIT_SIGNAL_RMS | synth.F_RESID_L2, B=3, T=1),
    # d = 1024: eight waves per block; a width that is not a power of two
    dict(d=1024, H=2, V=700, N=4, B=1, T=3),
    dict(d=192, H=3, V=500, N=4, B=1, T=4),
]


@pytest.mark.parametrize("var", CASES, ids=lambda v: "-".join(f"{k}{v[k]}" for k in v))
def test_fixed_iteration_solve_matches_per_iteration_update(oracle_lib, var):
    var = dict(var)
    B, T = var.pop("B"), var.pop("T")
    mc = synth.ModelConfig(r=32, **var)
    w = synth.make_token_sensitive_weights(mc, seed=5)
    toks = synth.make_tokens("uniform", B, T, mc.V, seed=2)
    be = GpuDeqBackend(mc, B, T)
    be.upload_weights(w)
    log(f"fixed-iteration solve {var} B={B} T={T}")
    fused = be.forward(toks, max_iters=7, eps=0.0, want=ALL)
    per_iter = be.forward(toks, max_iters=7, eps=1e-30, want=ALL)
    s_in = be.forward(s_in=np.ascontiguousarray(w["embed"][toks]), max_iters=7, eps=0.0, want=ALL)
    be.close()
    assert (fused["iters"] == 7).all() and not fused["converged"].any()
    for k in ALL:
        assert np.array_equal(fused[k], per_iter[k]), f"{k}: fused update differs from the update kernel"
        assert np.array_equal(fused[k], s_in[k]), f"{k}: s_in path differs"
    ref = oracle_lib.Oracle(dataclasses.replace(mc, max_iters=7, eps=0.0), w).forward(toks)
    assert_forward_parity(fused, ref, f"fixed {var}")
    assert np.array_equal(fused["argmax"], ref["argmax"])


@pytest.mark.parametrize("prec", ["bf16x3", "bf16", "fp32"])
def test_fixed_iteration_solve_every_gemm_arithmetic(oracle_lib, prec):
    """The same comparison in the other GEMM arithmetics (the fused update runs in the split
    products, bf16 halves included; with fp32 GEMMs every iteration runs the update kernel)."""
    flag = {"bf16x3": synth.F_GEMM_BF16X3, "bf16": synth.F_GEMM_BF16, "fp32": synth.F_GEMM_FP32}[prec]
    mc = synth.ModelConfig(d=256, H=4, V=600, N=4, r=32, flags=flag)
    w = synth.make_token_sensitive_weights(mc, seed=6)
    toks = synth.make_tokens("uniform", 1, 4, mc.V, seed=3)
    be = GpuDeqBackend(mc, 1, 4)
    be.upload_weights(w)
    log(f"fixed-iteration solve, {prec} GEMMs")
    fused = be.forward(toks, max_iters=6, eps=0.0, want=ALL)
    per_iter = be.forward(toks, max_iters=6, eps=1e-30, want=ALL)
    be.close()
    for k in ALL:
        assert np.array_equal(fused[k], per_iter[k]), f"{prec} {k}: fused update differs from the update kernel"
    if prec != "bf16":  # the bf16-input products are a reduced-precision variant
        ref = oracle_lib.Oracle(dataclasses.replace(mc, max_iters=6, eps=0.0), w).forward(toks)
        assert_forward_parity(fused, ref, f"fixed {prec}")
