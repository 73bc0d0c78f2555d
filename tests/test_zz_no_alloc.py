"""The allocation-free embed_context entry point against the allocating one, through the C ABI
(needs an MI355X).  Both run the same kernels, so the results must be bit-identical; the second
call is smaller than the first, so it also shows that what the first call left in the shared
per-device buffer does not leak into the next."""
import numpy as np
import pytest
# torch (device buffers) brings its own HIP runtime: imported before the library is first loaded
import torch

from aideen_amd import synth
from aideen_amd._lib import ADN_E_CAPACITY, AdnError
from aideen_amd.backend import GpuDeqBackend

pytestmark = pytest.mark.gpu


def log(msg):
    print(msg, flush=True)


@pytest.mark.parametrize("d", [128, 512, 2048])
def test_noalloc_equals_allocating_entry_point(d):
    mc = synth.ModelConfig(d=d, H=2, V=900, N=1, flags=0)
    w = synth.make_weights(mc, seed=11)
    dev = torch.device("cuda:0")
    be = GpuDeqBackend(mc, 6, 300)
    be.upload_weights(w)
    for B, T, ctx in [(6, 300, 64), (2, 37, 10)]:  # the second call is smaller
        log(f"noalloc d={d} B={B} T={T} ctx={ctx}")
        toks = torch.from_numpy(synth.make_tokens("uniform", B, T, mc.V, seed=B + T)).to(dev)
        ref = torch.full((B, T, d), float("nan"), dtype=torch.float32, device=dev)
        got = torch.full((B, T, d), float("nan"), dtype=torch.float32, device=dev)
        be.embed_context_async(toks, ctx, ref)
        be.embed_context_noalloc(toks, ctx, got)
        be.synchronize()
        r, g = ref.cpu().numpy(), got.cpu().numpy()
        assert np.isfinite(r).all()
        assert np.array_equal(g, r)
    be.close()


def test_noalloc_rejects_requests_beyond_its_buffer():
    """2 * 1 * ceil(4100 / 4) * 2048 doubles > 4194304: refused before anything is launched."""
    log("noalloc capacity")
    mc = synth.ModelConfig(d=2048, H=1, V=50, N=1, flags=0)
    be = GpuDeqBackend(mc, 1, 4100)
    be.upload_weights(synth.make_weights(mc, seed=1))
    dev = torch.device("cuda:0")
    toks = torch.zeros((1, 4100), dtype=torch.int32, device=dev)
    out = torch.empty((1, 4100, 2048), dtype=torch.float32, device=dev)
    with pytest.raises(AdnError) as ei:
        be.embed_context_noalloc(toks, 16, out)
    assert ei.value.code == ADN_E_CAPACITY
    small = toks[:, :4096].contiguous()
    be.embed_context_noalloc(small, 16, out[:, :4096])  # exactly the buffer's size
    be.synchronize()
    assert np.isfinite(out[:, :4096].cpu().numpy()).all()
    be.close()


def test_noalloc_overlap_is_reported():
    """Overlapping calls on one GPU race on the shared array; the library detects them.  The
    overlap is forced from the host: with the guard's count of calls in flight set to 1 (as if
    another call were running), a call reports the overlap on the context's next blocking call;
    with the count back at 0, calls in stream order report nothing, and leave the count at 0."""
    log("noalloc overlap guard")
    mc = synth.ModelConfig(d=128, H=2, V=300, N=1, flags=0)
    be = GpuDeqBackend(mc, 2, 40)
    be.upload_weights(synth.make_weights(mc, seed=2))
    dev = torch.device("cuda:0")
    toks_h = synth.make_tokens("uniform", 2, 40, mc.V, seed=3)
    toks = torch.from_numpy(toks_h).to(dev)
    out = torch.empty((2, 40, 128), dtype=torch.float32, device=dev)
    be.noalloc_guard_set(1)
    be.embed_context_noalloc(toks, 8, out)
    with pytest.raises(AdnError, match="overlapped"):
        be.forward(toks_h, want=("iters",))
    be.noalloc_guard_set(0)
    for _ in range(3):
        be.embed_context_noalloc(toks, 8, out)
    be.forward(toks_h, want=("iters",))  # no error: the calls ran in stream order
    ref = torch.empty_like(out)
    be.embed_context_async(toks, 8, ref)
    be.synchronize()
    assert np.array_equal(out.cpu().numpy(), ref.cpu().numpy())
    be.close()
