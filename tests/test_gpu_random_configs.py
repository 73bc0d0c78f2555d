"""Seeded random configurations against the oracle (needs an MI355X).

Each case draws a width, slot count, vocabulary, carrier, flag set (init rule, score clamp,
anchor-excluding RMS, residual norm, W_in orientation, selective carrier, q/k bias), GEMM
arithmetic, Anderson depth, batch shape, tolerance and iteration cap, so that the kernel paths
chosen by size (few-token attention inside W_o, the fixed-iteration update inside Q|K|V, the pool
inside the last update, skinny and tiled products, per-step and matrix-form scans) meet every
switch of the forward spec (fixed_point_memory_reasoning.rs:1300-1486) in combinations no
hand-written case lists.  Every output of every token is compared with the oracle on the
token-sensitive weights.  With Anderson mixing the tolerance is 0 (the residual is not
monotone, so an exit near eps can move by two iterations; every iteration then runs), as it is
in the fixed-iteration cases.
"""
import numpy as np
import pytest

from aideen_amd import synth
from aideen_amd.backend import GpuDeqBackend
from test_gpu_parity import assert_forward_parity, log

pytestmark = pytest.mark.gpu

ALL = ("h_star", "pooled", "logits", "argmax", "iters", "converged", "scan_y", "scan_state")


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
    ref = oracle_lib.Oracle(mc, w).forward(toks, nthreads=16)
    assert_forward_parity(got, ref, f"random config {seed}")
    if mc.eps == 0.0:
        assert (got["iters"] == mc.max_iters).all()
