"""A reference-layout .aidn checkpoint loaded by the library and run on the GPU, against the
oracle on the same model (needs an MI355X).  Bar as for the forward: rtol 1e-4 / atol 1e-3,
iterations within +-1."""
import dataclasses

import numpy as np
import pytest

from aideen_amd import aidn, synth
from aideen_amd.backend import GpuDeqBackend

pytestmark = pytest.mark.gpu


def log(msg):
    print(msg, flush=True)


def shared_model(mc, seed=3):
    w = dict(synth.make_weights(mc, seed=seed))
    for n in ("w_q", "w_k", "w_v", "w_o", "w_in", "w_out", "wx_diag", "b_delta"):
        w[n] = np.ascontiguousarray(np.repeat(w[n][:1], mc.H, axis=0))
    w.update(synth.make_hist_weights(mc, seed=seed, strong=True))
    return w


@pytest.mark.parametrize("memory", [False, True], ids=["canonical", "memory"])
def test_checkpoint_forward_matches_oracle(oracle_lib, tmp_path, memory):
    log(f"aidn checkpoint memory={memory}")
    mc = synth.ModelConfig(d=128, H=4, V=400, N=1, r=32, flags=0, qk_bias=True, max_iters=14, eps=1e-4)
    w = shared_model(mc)
    cfg, ex, meta = aidn.reference_export(mc, w, damping=0.7)
    p = str(tmp_path / "m.aidn")
    aidn.write_aidn(p, cfg, ex, meta)
    flags = synth.F_MEMORY if memory else 0
    B, T = 2, 9
    be = GpuDeqBackend.from_aidn(p, max_batch=B, max_seq=T, flags=flags)
    assert be.model.max_iters == 14 and be.model.d == 128 and be.model.H == 4
    toks = synth.make_tokens("uniform", B, T, mc.V, seed=6)
    got = be.forward(toks)
    mo = dataclasses.replace(mc, flags=flags)
    o = oracle_lib.Oracle(mo, w)
    ref = o.forward_memory(toks) if memory else o.forward(toks)
    for k in ("h_star", "pooled", "logits"):
        np.testing.assert_allclose(got[k], ref[k], rtol=1e-4, atol=1e-3, err_msg=k)
    assert np.abs(got["iters"].astype(int) - ref["iters"].astype(int)).max() <= 1
    if memory:
        np.testing.assert_allclose(got["scan_y"], ref["m_seq"], rtol=1e-4, atol=1e-3)
