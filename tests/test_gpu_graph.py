"""The device-memory forward captured in a HIP graph (needs an MI355X).

adn_forward_async enqueues kernels and device-to-device copies only: the Picard loop's active
count stays on the device, the per-forward resets (bounds, counts) are kernels rather than
memsets, and nothing is allocated once a first call has sized the context.  So a caller can
capture one forward into a graph and replay it.  Each case runs the forward eagerly, captures the
same call, and replays the graph three times with other eager work and synchronisations between
the replays (the outputs overwritten with a sentinel before each); every replay must equal the
eager outputs bit for bit (every kernel here computes each token's values independently of the
order of the active list, so the results are deterministic).
"""
import numpy as np
import pytest

from aideen_amd import synth
from aideen_amd.backend import GpuDeqBackend

pytestmark = pytest.mark.gpu


def log(msg):
    print(msg, flush=True)


def capture_and_replay(mc, w, B, T, toks):
    import torch
    dev = torch.device("cuda:0")
    be = GpuDeqBackend(mc, B, T)
    be.upload_weights(w)
    stream = torch.cuda.Stream(dev)
    be.set_stream(stream.cuda_stream)
    with torch.cuda.stream(stream):
        tok_d = torch.from_numpy(toks).to(dev)
        outs = dict(h_star=torch.empty((B, T, mc.H, mc.d), device=dev),
                    iters=torch.empty((B, T), dtype=torch.int32, device=dev),
                    converged=torch.empty((B, T), dtype=torch.int32, device=dev),
                    pooled=torch.empty((B, T, mc.d), device=dev),
                    logits=torch.empty((B, T, mc.V), device=dev),
                    argmax=torch.empty((B, T), dtype=torch.int32, device=dev),
                    scan_y=torch.empty((B, T, mc.H, mc.d), device=dev),
                    scan_state=torch.empty((B, mc.H, mc.d, mc.N), device=dev))
        be.forward_async(tok_d, outputs=outs)
    torch.cuda.synchronize()
    be.synchronize()
    ref = {k: v.clone() for k, v in outs.items()}
    assert np.isfinite(ref["h_star"].cpu().numpy()).all()

    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        be.forward_async(tok_d, outputs=outs)
    torch.cuda.synchronize()
    for rep in range(3):
        with torch.cuda.stream(stream):
            for v in outs.values():
                v.fill_(7)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for k in outs:
            assert torch.equal(outs[k], ref[k]), f"replay {rep}: {k} differs from the eager forward"
        x = torch.randn(1 << 20, device=dev)
        assert (x * 2).sum().item() == pytest.approx(2 * x.sum().item(), rel=1e-4, abs=1e-2)
    be.synchronize()
    log(f"  3 replays identical to the eager forward (mean iterations {ref['iters'].float().mean().item():.2f})")


@pytest.mark.parametrize("anderson_m", [0, 3])
def test_forward_graph_replays_match_eager(anderson_m):
    """1200 tokens at d = 512, H = 2, V = 700: the Q|K|V, W_o and LM-head GEMMs on the persistent
    256x256 tiles (W_o and the LM head reading operands their producers wrote pre-split), the
    device-side active list, the carrier scan and the readout; with and without Anderson mixing."""
    log(f"graph capture, canonical forward, anderson m={anderson_m}")
    mc = synth.ModelConfig(d=512, H=2, V=700, N=4, r=32, anderson_m=anderson_m, max_iters=20)
    w = synth.make_weights(mc, seed=5)
    B, T = 4, 300
    toks = synth.make_tokens("zipf", B, T, mc.V, seed=6)
    capture_and_replay(mc, w, B, T, toks)


def test_forward_graph_wide_rows_anderson_replays_match_eager():
    """Rows of 1024 floats with Anderson mixing: the fused update and mix for wide rows (a lane's
    elements walked in groups, the rows in dynamic LDS, the per-token mix coefficients kept between
    iterations) captured in the graph with the rest of the forward."""
    log("graph capture, canonical forward, d=1024, anderson m=4")
    mc = synth.ModelConfig(d=1024, H=2, V=600, N=4, r=32, anderson_m=4, max_iters=12)
    w = synth.make_weights(mc, seed=15)
    B, T = 2, 520
    toks = synth.make_tokens("zipf", B, T, mc.V, seed=16)
    capture_and_replay(mc, w, B, T, toks)


def test_memory_forward_graph_replays_match_eager():
    """The memory-coupled forward (positions in order, the per-position Picard loops, the history
    context and the carrier state copied between buffers on the device) captured whole."""
    log("graph capture, memory-coupled forward")
    mc = synth.ModelConfig(d=256, H=4, V=500, N=1, r=32, flags=synth.F_MEMORY, max_iters=12)
    w = dict(synth.make_weights(mc, seed=7))
    w.update(synth.make_hist_weights(mc, seed=8, strong=True))
    B, T = 3, 10
    toks = synth.make_tokens("uniform", B, T, mc.V, seed=9)
    capture_and_replay(mc, w, B, T, toks)


def test_serving_step_graph_with_noalloc_embed():
    """A serving step that allocates nothing, captured whole: the queries of every position from
    the token windows (adn_embed_context_noalloc, whose totals live in the library's fixed device
    buffer) and the forward on those queries (logits, arg-max, h*).  The graph reads the token ids
    from device memory at each replay: replays on two different token sets, written into the
    captured input buffer between replays, must each equal the eager step on those tokens."""
    import torch
    log("graph capture, embed_context_noalloc + forward on the queries")
    mc = synth.ModelConfig(d=512, H=2, V=700, N=4, r=32, max_iters=20)
    w = synth.make_weights(mc, seed=12)
    B, T, ctx = 4, 300, 64
    dev = torch.device("cuda:0")
    be = GpuDeqBackend(mc, B, T)
    be.upload_weights(w)
    stream = torch.cuda.Stream(dev)
    be.set_stream(stream.cuda_stream)
    token_sets = [torch.from_numpy(synth.make_tokens("zipf", B, T, mc.V, seed=s)).to(dev) for s in (13, 14)]
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        tok = torch.empty((B, T), dtype=torch.int32, device=dev)
        q = torch.empty((B, T, mc.d), device=dev)
        outs = dict(h_star=torch.empty((B, T, mc.H, mc.d), device=dev),
                    iters=torch.empty((B, T), dtype=torch.int32, device=dev),
                    logits=torch.empty((B, T, mc.V), device=dev),
                    argmax=torch.empty((B, T), dtype=torch.int32, device=dev))

    def step():
        be.embed_context_noalloc(tok, ctx, q)
        be.forward_async(s_in=q, outputs=outs)

    refs = []
    for ts in token_sets:
        with torch.cuda.stream(stream):
            tok.copy_(ts)
            step()
        torch.cuda.synchronize()
        be.synchronize()
        refs.append({k: v.clone() for k, v in outs.items()})
    assert not torch.equal(refs[0]["argmax"], refs[1]["argmax"])

    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        step()
    torch.cuda.synchronize()
    for rep, i in enumerate((1, 0, 1)):
        with torch.cuda.stream(stream):
            tok.copy_(token_sets[i])
            q.fill_(7)
            for v in outs.values():
                v.fill_(7)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for k in outs:
            assert torch.equal(outs[k], refs[i][k]), f"replay {rep} (token set {i}): {k} differs from the eager step"
    be.synchronize()
    be.close()
    log("  replays on two token sets identical to the eager steps")
