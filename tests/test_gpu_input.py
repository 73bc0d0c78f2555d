"""Input pipeline on the HIP path vs the CPU oracle, through the C ABI (needs an MI355X).

embed_context (tokenizer.rs:133-149) for the window ending at every position, as the trainer
builds the query of each position (trainer.rs:4690-4696).  The GPU sums in fp64 prefix form,
the oracle (like the reference) in fp32 window order, so the bar is a tolerance: atol 2e-6 on
the unit-norm outputs against the oracle, 1e-6 against a float64 brute force.
"""
import numpy as np
import pytest
# torch (device buffers for the async form) brings its own HIP runtime: imported before the
# library is first loaded so that one runtime serves both
import torch

from aideen_amd import synth
from aideen_amd._lib import AdnError
from aideen_amd.backend import GpuDeqBackend

pytestmark = pytest.mark.gpu


def log(msg):
    print(msg, flush=True)


def f64_embed_context(E, toks, ctx):
    B, T = toks.shape
    out = np.zeros((B, T, E.shape[1]))
    for b in range(B):
        for i in range(T):
            s = max(0, i - ctx + 1)
            win = toks[b, s:i + 1]
            w = np.arange(1, len(win) + 1, dtype=np.float64) / len(win)
            r = (E[win].astype(np.float64) * w[:, None]).sum(0)
            n = np.sqrt((r * r).sum())
            out[b, i] = r / n if n > 1e-6 else r
    return out


CASES = [
    dict(d=64, V=300, B=2, T=37, ctx=16),    # sliding windows, ragged chunk
    dict(d=128, V=500, B=3, T=70, ctx=70),   # prefix windows only
    dict(d=512, V=2000, B=2, T=100, ctx=33),  # ctx not a multiple of the chunk
    dict(d=256, V=400, B=1, T=65, ctx=1),    # every position its own row
    dict(d=2048, V=300, B=2, T=40, ctx=256),  # widest rows
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "-".join(f"{k}{c[k]}" for k in c))
def test_embed_context_matches_oracle(oracle_lib, case):
    log(f"embed_context {case}")
    mc = synth.ModelConfig(d=case["d"], H=2, V=case["V"], N=1, flags=0)
    w = synth.make_weights(mc, seed=2)
    toks = synth.make_tokens("uniform", case["B"], case["T"], mc.V, seed=3)
    be = GpuDeqBackend(mc, case["B"], case["T"])
    be.upload_weights(w)
    got = be.embed_context(toks, case["ctx"])
    ref = oracle_lib.embed_context(w["embed"], toks, case["ctx"])
    np.testing.assert_allclose(got, ref, rtol=0, atol=2e-6)
    np.testing.assert_allclose(got, f64_embed_context(w["embed"], toks, case["ctx"]), rtol=0, atol=1e-6)


def test_embed_context_feeds_the_forward(oracle_lib):
    """Tokens -> embed_context -> the canonical forward on s_in, on the GPU and in the oracle
    (whose forward reads its inputs from an embedding table: the queries become that table)."""
    log("embed_context -> forward")
    mc = synth.ModelConfig(d=128, H=4, V=500, N=16)
    w = synth.make_weights(mc, seed=4)
    B, T, ctx = 2, 24, 10
    toks = synth.make_tokens("uniform", B, T, mc.V, seed=5)
    be = GpuDeqBackend(mc, B, T)
    be.upload_weights(w)
    q = be.embed_context(toks, ctx)
    got = be.forward(s_in=q)
    qref = oracle_lib.embed_context(w["embed"], toks, ctx)
    w2 = dict(w)
    w2["embed"] = qref.reshape(B * T, mc.d)
    ref = oracle_lib.Oracle(mc, w2).forward(np.arange(B * T, dtype=np.int32).reshape(B, T))
    for k in ("h_star", "pooled"):
        np.testing.assert_allclose(got[k], ref[k], rtol=1e-4, atol=1e-3, err_msg=k)
    assert np.abs(got["iters"].astype(int) - ref["iters"].astype(int)).max() <= 1


def test_embed_context_async_equals_blocking():
    log("embed_context async")
    mc = synth.ModelConfig(d=256, H=2, V=700, N=1, flags=0)
    w = synth.make_weights(mc, seed=6)
    B, T = 4, 50
    toks = synth.make_tokens("zipf", B, T, mc.V, seed=7)
    be = GpuDeqBackend(mc, B, T)
    be.upload_weights(w)
    ref = be.embed_context(toks, 20)
    dev = torch.device("cuda:0")
    out = torch.empty((B, T, mc.d), dtype=torch.float32, device=dev)
    be.embed_context_async(torch.from_numpy(toks).to(dev), 20, out)
    be.synchronize()
    assert np.array_equal(out.cpu().numpy(), ref)


def test_embed_context_errors():
    log("embed_context errors")
    mc = synth.ModelConfig(d=64, H=2, V=100, N=1, flags=0)
    be = GpuDeqBackend(mc, 2, 8)
    toks = np.zeros((2, 8), np.int32)
    with pytest.raises(AdnError):
        be.embed_context(toks, 4)  # no weights yet
    be.upload_weights(synth.make_weights(mc, seed=1))
    with pytest.raises(AdnError, match="max_ctx"):
        be.embed_context(toks, 0)
    bad = toks.copy()
    bad[1, 3] = 100
    with pytest.raises(AdnError, match="vocab"):
        be.embed_context(bad, 4)
    with pytest.raises(AdnError, match="capacity"):
        be.embed_context(np.zeros((3, 8), np.int32), 4)
    assert be.embed_context(toks, 4).shape == (2, 8, 64)
