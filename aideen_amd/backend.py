"""Host-side mirror of the reference's GPU backend surfaces, over the C ABI.

Names, argument meaning and error behaviour follow the Rust API this path replaces:

* ``GpuDeqBackend`` -- ``aideen-backbone/src/gpu_deq.rs:80-219``: ``new_blocking`` returns
  ``None`` when no GPU is present (:3122-3124), ``upload_weights`` (:3529-3667),
  ``reset_state`` (:3127-3164), ``run_forward_deq`` returning ``(h_next, iters)``
  (:3687-3727), ``run_forward_deq_pooled`` (:3729-3768), readbacks ``read_hnext_seq`` /
  ``read_hpooled_seq`` (:5833-5894) and the exact logits of
  ``GpuLmHeadTrainer::read_exact_logits_from_h`` (gpu_lm_head.rs:1813-1879).
* ``HipBlockBackend.fpm_batch_step`` -- ``BlockBackend`` (aideen-core/src/block_backend.rs:22-31).
* ``HipComputeBackend`` -- ``ComputeBackend`` (aideen-core/src/compute.rs:11-23).

Failures raise ``AdnError`` carrying the library's message (the Rust side returns
``Err(&'static str)`` / ``Err(String)``).
"""
from __future__ import annotations

import ctypes as C
import os
from typing import Dict, Optional

import numpy as np

from . import _lib
from ._lib import AdnConfig, AdnOutputs, AdnRun, AdnWeights, check, lib

_F32P = _lib.F32P
_I32P = _lib.I32P


def _fp(a: Optional[np.ndarray]):
    if a is None:
        return None
    assert a.dtype == np.float32 and a.flags["C_CONTIGUOUS"], "float32 C-contiguous array expected"
    return a.ctypes.data_as(_F32P)


def _ip(a: Optional[np.ndarray]):
    if a is None:
        return None
    assert a.dtype == np.int32 and a.flags["C_CONTIGUOUS"], "int32 C-contiguous array expected"
    return a.ctypes.data_as(_I32P)


def _dev_f(t) -> Optional[C.POINTER(C.c_float)]:
    return None if t is None else C.cast(C.c_void_p(t.data_ptr()), _F32P)


def _dev_i(t) -> Optional[C.POINTER(C.c_int32)]:
    return None if t is None else C.cast(C.c_void_p(t.data_ptr()), _I32P)


def device_count() -> int:
    n = C.c_int32(0)
    check(lib().adn_device_count(C.byref(n)))
    return n.value


class GpuDeqBackend:
    """One context on the current HIP device (single-threaded, like the reference backend)."""

    def __init__(self, model, max_batch: int, max_seq: int):
        self.model = model
        cfg = AdnConfig(model.d, model.H, model.V, model.N, model.r, max_batch, max_seq,
                        model.anderson_m, model.flags)
        self._ctx = C.c_void_p()
        check(lib().adn_create(C.byref(cfg), C.byref(self._ctx)))
        self.max_batch, self.max_seq = max_batch, max_seq
        self._weights_keepalive = None

    @classmethod
    def new_blocking(cls, model, max_batch: int = 1, max_seq: int = 1) -> Optional["GpuDeqBackend"]:
        """``None`` when no GPU is present (gpu_deq.rs:3122-3124)."""
        try:
            return cls(model, max_batch, max_seq)
        except _lib.AdnError as e:
            if e.code == _lib.ADN_E_NO_DEVICE:
                return None
            raise

    @classmethod
    def from_aidn(cls, path: str, max_batch: int = 1, max_seq: Optional[int] = None, flags: int = 0,
                  anderson_m: int = 0) -> "GpuDeqBackend":
        """A context for a reference checkpoint (the trainer's load_full, trainer.rs:6598-6680):
        the library's loader maps the file onto its weights; the model's max_deq_iters,
        deq_epsilon and damping become the run defaults."""
        import dataclasses
        from .aidn import AidnModel
        from .synth import ModelConfig
        m = AidnModel(path)
        w, cfg, run = m.weights()
        m.close()
        mc = ModelConfig(d=cfg["d_r"], H=cfg["h_slots"], V=cfg["vocab"], N=cfg["d_state"], r=cfg["rank"],
                         flags=flags, max_iters=run["max_iters"], eps=run["eps"], beta=run["damping"],
                         anderson_m=anderson_m)
        be = cls(mc, max_batch, max_seq or cfg["max_seq"])
        be.upload_weights(w)
        return be

    def close(self) -> None:
        if self._ctx:
            lib().adn_destroy(self._ctx)
            self._ctx = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # ------------------------------------------------------------------------------------
    def set_stream(self, stream_handle: Optional[int]) -> None:
        check(lib().adn_set_stream(self._ctx, C.c_void_p(stream_handle) if stream_handle else None))

    def synchronize(self) -> None:
        check(lib().adn_synchronize(self._ctx))

    def upload_weights(self, w: Dict[str, Optional[np.ndarray]], layout: int = _lib.ADN_LAYOUT_OUT_IN) -> None:
        keep = {k: (None if v is None else np.ascontiguousarray(v, dtype=np.float32)) for k, v in w.items()}
        cw = AdnWeights(**{k: _fp(keep.get(k)) for k in _lib.WEIGHT_FIELDS})
        check(lib().adn_upload_weights(self._ctx, C.byref(cw), layout))
        self._weights_keepalive = keep

    def reset_state(self) -> None:
        check(lib().adn_reset_state(self._ctx))

    # ------------------------------------------------------------------------------------
    def forward(self, tokens: Optional[np.ndarray] = None, s_in: Optional[np.ndarray] = None, *,
                max_iters: Optional[int] = None, eps: Optional[float] = None,
                damping: Optional[float] = None, want=("h_star", "pooled", "logits", "argmax", "iters",
                                                        "scan_y", "scan_state", "converged"),
                scan_state_in: Optional[np.ndarray] = None) -> Dict[str, np.ndarray]:
        """Host-memory forward (blocking).  Returns the requested outputs."""
        m = self.model
        if tokens is not None:
            tokens = np.ascontiguousarray(tokens, dtype=np.int32)
            B, T = tokens.shape
        else:
            s_in = np.ascontiguousarray(s_in, dtype=np.float32)
            B, T = s_in.shape[:2]
        run = AdnRun(B, T, m.max_iters if max_iters is None else max_iters,
                     m.eps if eps is None else eps, m.beta if damping is None else damping,
                     _ip(tokens), _fp(s_in),
                     _fp(None if scan_state_in is None else np.ascontiguousarray(scan_state_in, np.float32)))
        shapes = dict(h_star=((B, T, m.H, m.d), np.float32), pooled=((B, T, m.d), np.float32),
                      logits=((B, T, m.V), np.float32), argmax=((B, T), np.int32),
                      iters=((B, T), np.int32), scan_y=((B, T, m.H, m.d), np.float32),
                      scan_state=((B, m.H, m.d, m.N), np.float32), converged=((B, T), np.int32))
        outs = {k: np.zeros(*shapes[k]) for k in want}
        co = AdnOutputs(**{k: (_fp(v) if v.dtype == np.float32 else _ip(v)) for k, v in outs.items()})
        check(lib().adn_forward(self._ctx, C.byref(run), C.byref(co)))
        return outs

    def forward_async(self, tokens=None, s_in=None, *, outputs: Dict[str, object],
                      max_iters: Optional[int] = None, eps: Optional[float] = None,
                      damping: Optional[float] = None, scan_state_in=None) -> None:
        """Device-memory forward (enqueue only).  ``tokens`` / ``s_in`` / outputs are torch
        tensors on the GPU (anything with ``data_ptr()``)."""
        m = self.model
        if tokens is not None:
            B, T = tokens.shape
        else:
            B, T = s_in.shape[:2]
        run = AdnRun(B, T, m.max_iters if max_iters is None else max_iters,
                     m.eps if eps is None else eps, m.beta if damping is None else damping,
                     _dev_i(tokens), _dev_f(s_in), _dev_f(scan_state_in))
        co = AdnOutputs(h_star=_dev_f(outputs.get("h_star")), pooled=_dev_f(outputs.get("pooled")),
                        logits=_dev_f(outputs.get("logits")), argmax=_dev_i(outputs.get("argmax")),
                        iters=_dev_i(outputs.get("iters")), scan_y=_dev_f(outputs.get("scan_y")),
                        scan_state=_dev_f(outputs.get("scan_state")),
                        converged=_dev_i(outputs.get("converged")))
        check(lib().adn_forward_async(self._ctx, C.byref(run), C.byref(co)))

    def profile_forward(self, tokens=None, s_in=None, *, outputs: Dict[str, object],
                        max_iters: Optional[int] = None, eps: Optional[float] = None,
                        damping: Optional[float] = None) -> dict:
        """One device-memory forward with a HIP event pair around every kernel; returns per-stage
        device time, algorithmic FLOPs/bytes, launch counts and the active tokens per iteration."""
        m = self.model
        B, T = (tokens.shape if tokens is not None else s_in.shape[:2])
        run = AdnRun(B, T, m.max_iters if max_iters is None else max_iters,
                     m.eps if eps is None else eps, m.beta if damping is None else damping,
                     _dev_i(tokens), _dev_f(s_in), None)
        co = AdnOutputs(h_star=_dev_f(outputs.get("h_star")), pooled=_dev_f(outputs.get("pooled")),
                        logits=_dev_f(outputs.get("logits")), argmax=_dev_i(outputs.get("argmax")),
                        iters=_dev_i(outputs.get("iters")), scan_y=_dev_f(outputs.get("scan_y")),
                        scan_state=_dev_f(outputs.get("scan_state")),
                        converged=_dev_i(outputs.get("converged")))
        prof = _lib.AdnProfile()
        check(lib().adn_profile_forward(self._ctx, C.byref(run), C.byref(co), C.byref(prof)))
        stages = {}
        for i, name in enumerate(_lib.STAGES):
            if prof.launches[i]:
                stages[name] = dict(ms=prof.ms[i], flops=prof.flops[i], bytes=prof.bytes[i],
                                    launches=prof.launches[i])
        return dict(stages=stages, active=list(prof.active[:prof.n_iters]), total_ms=prof.total_ms)

    # input pipeline --------------------------------------------------------------------------
    def embed_context(self, tokens: np.ndarray, max_ctx: int) -> np.ndarray:
        """``Tokenizer::embed_context`` (tokenizer.rs:133-149) for the window ending at every
        position (trainer.rs:4690-4696): tokens [B][T] -> queries [B][T][d], an ``s_in``."""
        tokens = np.ascontiguousarray(tokens, dtype=np.int32)
        B, T = tokens.shape
        out = np.zeros((B, T, self.model.d), np.float32)
        check(lib().adn_embed_context(self._ctx, B, T, _ip(tokens), int(max_ctx), _fp(out)))
        return out

    def embed_context_async(self, tokens, max_ctx: int, out) -> None:
        """Device-memory form (torch tensors): enqueue only."""
        B, T = tokens.shape
        check(lib().adn_embed_context_async(self._ctx, B, T, _dev_i(tokens), int(max_ctx), _dev_f(out)))

    def embed_context_noalloc(self, tokens, max_ctx: int, out) -> None:
        """Device-memory form that allocates nothing (a fixed per-device buffer; concurrent calls
        on one GPU race): enqueue only."""
        B, T = tokens.shape
        check(lib().adn_embed_context_noalloc(self._ctx, B, T, _dev_i(tokens), int(max_ctx), _dev_f(out)))

    def noalloc_guard_set(self, calls_in_flight: int) -> None:
        """Diagnostics: set this GPU's count of embed_context_noalloc calls in flight (tests force
        an overlap with it)."""
        check(lib().adn_noalloc_guard_set(self._ctx, int(calls_in_flight)))

    # backward ----------------------------------------------------------------------------------
    def adjoint(self, dl: np.ndarray, iters: int, damping: Optional[float] = None,
                h_star: Optional[np.ndarray] = None):
        """The clean adjoint Picard for the tokens of the most recent forward (gpu_deq.rs:4736-4975):
        dl [B][T][d] = dL/d pooled h* -> (v [B][T][H][d], source gradient [B][T][d])."""
        m = self.model
        dl = np.ascontiguousarray(dl, np.float32)
        lead = dl.shape[:-1]
        ntok = int(np.prod(lead))
        v = np.zeros(lead + (m.H, m.d), np.float32)
        src = np.zeros(lead + (m.d,), np.float32)
        hs = None if h_star is None else np.ascontiguousarray(h_star, np.float32)
        check(lib().adn_adjoint(self._ctx, ntok, _fp(hs), _fp(dl), int(iters),
                                m.beta if damping is None else float(damping), _fp(v), _fp(src)))
        return v, src

    def adjoint_async(self, ntok: int, dl, iters: int, damping: float, v_out=None, src_out=None,
                      h_star=None) -> None:
        check(lib().adn_adjoint_async(self._ctx, int(ntok), _dev_f(h_star), _dev_f(dl), int(iters), float(damping),
                                      _dev_f(v_out), _dev_f(src_out)))

    # reference-named conveniences ---------------------------------------------------------
    def run_forward_deq(self, batch, seq, max_iters, eps, damping, s_in):
        """``run_forward_deq`` (gpu_deq.rs:3687-3727): H_next [B*T*H*d] and iteration counts."""
        s = np.asarray(s_in, np.float32).reshape(batch, seq, self.model.d)
        o = self.forward(s_in=s, max_iters=max_iters, eps=eps, damping=damping, want=("h_star", "iters"))
        return o["h_star"].reshape(-1), o["iters"].reshape(-1).astype(np.uint32)

    def run_forward_deq_pooled(self, batch, seq, max_iters, eps, damping, s_in):
        """``run_forward_deq_pooled`` (gpu_deq.rs:3729-3768): pooled [B*T*d] and iteration counts."""
        s = np.asarray(s_in, np.float32).reshape(batch, seq, self.model.d)
        o = self.forward(s_in=s, max_iters=max_iters, eps=eps, damping=damping, want=("pooled", "iters"))
        return o["pooled"].reshape(-1), o["iters"].reshape(-1).astype(np.uint32)

    def decode_greedy(self, prompt, n_new: int, ctx_len: int, *, max_iters: int = 10, eps: float = 0.0,
                      damping: Optional[float] = None, repetition_penalty: float = 1.0) -> np.ndarray:
        """``Trainer::generate`` with greedy sampling (trainer.rs:4219-4431): prompt [B][T0] ->
        the n_new appended token ids [B][n_new].  The defaults are generate's own solve (10 Picard
        steps, no early exit); ``ctx_len`` is ``ArchitectureConfig::ctx_len``."""
        prompt = np.ascontiguousarray(prompt, dtype=np.int32)
        if prompt.ndim == 1:
            prompt = prompt[:, None]
        B, T0 = prompt.shape
        out = np.zeros((B, n_new), np.int32)
        check(lib().adn_decode_greedy(self._ctx, B, T0, _ip(prompt), int(n_new), int(ctx_len), int(max_iters),
                                      float(eps), self.model.beta if damping is None else float(damping),
                                      float(repetition_penalty), _ip(out)))
        return out

    def decode_sample(self, prompt, n_new: int, ctx_len: int, *, temperature: float, top_p: float, top_k: int,
                      repetition_penalty: float = 1.0, uniforms=None, seed: Optional[int] = None,
                      max_iters: int = 10, eps: float = 0.0, damping: Optional[float] = None) -> np.ndarray:
        """``Trainer::generate`` (trainer.rs:4219-4431) with ``LmHead::sample``'s temperature, top_p,
        top_k and repetition penalty (lm_head.rs:78-168).  The reference draws each step's uniform from
        ``thread_rng``; here ``uniforms`` [B][n_new] in [0, 1) are the draws (or, when None, 24-bit
        draws as ``rng.gen::<f32>()`` makes them, from a numpy generator seeded with ``seed``)."""
        prompt = np.ascontiguousarray(prompt, dtype=np.int32)
        if prompt.ndim == 1:
            prompt = prompt[:, None]
        B, T0 = prompt.shape
        if uniforms is None:
            rng = np.random.default_rng(seed)
            uniforms = (rng.integers(0, 1 << 24, size=(B, n_new)) * 2.0 ** -24).astype(np.float32)
        uni = np.ascontiguousarray(uniforms, np.float32).reshape(B, n_new)
        out = np.zeros((B, n_new), np.int32)
        check(lib().adn_decode_sample(self._ctx, B, T0, _ip(prompt), int(n_new), int(ctx_len), int(max_iters),
                                      float(eps), self.model.beta if damping is None else float(damping),
                                      float(temperature), float(top_p), int(top_k), float(repetition_penalty),
                                      _fp(uni), _ip(out)))
        return out

    def lm_sample(self, logits, uniforms, *, temperature: float, top_p: float, top_k: int,
                  repetition_penalty: float = 1.0, context=None) -> np.ndarray:
        """``LmHead::sample`` (lm_head.rs:78-168) on rows of logits [rows][V] with the draws
        ``uniforms`` [rows]; ``context`` is a list of each row's context token ids (or None)."""
        lg = np.ascontiguousarray(logits, np.float32)
        if lg.ndim == 1:
            lg = lg[None, :]
        rows, V = lg.shape
        uni = np.ascontiguousarray(uniforms, np.float32).reshape(rows)
        if context is None:
            ctx = np.zeros((rows, 0), np.int32)
            lens = np.zeros(rows, np.int32)
        else:
            width = max(1, max(len(c) for c in context))
            ctx = np.zeros((rows, width), np.int32)
            lens = np.array([len(c) for c in context], np.int32)
            for i, c in enumerate(context):
                ctx[i, :len(c)] = c
        out = np.zeros(rows, np.int32)
        check(lib().adn_lm_sample(self._ctx, rows, V, _fp(lg), _ip(ctx), ctx.shape[1], _ip(lens), float(temperature),
                                  float(top_p), int(top_k), float(repetition_penalty), _fp(uni), _ip(out)))
        return out

    # weight preparation --------------------------------------------------------------------
    def spectral_norm(self, w: np.ndarray, n_iter: int = 20) -> float:
        w = np.ascontiguousarray(w, np.float32)
        s = C.c_float(0.0)
        check(lib().adn_spectral_norm(self._ctx, _fp(w), w.shape[0], w.shape[1], n_iter, C.byref(s)))
        return s.value

    def normalize_if_needed(self, w: np.ndarray, threshold: float, n_iter: int = 20) -> np.ndarray:
        w = np.ascontiguousarray(w, np.float32).copy()
        check(lib().adn_normalize_if_needed(self._ctx, _fp(w), w.shape[0], w.shape[1], threshold, n_iter))
        return w

    @staticmethod
    def _env_f32(name: str) -> Optional[float]:
        v = os.environ.get(name)
        try:
            return float(v) if v is not None else None
        except ValueError:
            return None

    def renormalize_spectral(self, n_iters: int = 12) -> np.ndarray:
        """GpuDeqBackend::renormalize_spectral (gpu_deq.rs:5567-5591): the uploaded block matrices
        renormalised on the device with the reference's thresholds and their environment overrides
        (AIDEEN_DEQ_ATTN_THRESHOLD 0.10 for W_q/W_k, AIDEEN_DEQ_WIN_THRESHOLD 0.30 for W_in,
        AIDEEN_DEQ_WV_THRESHOLD and AIDEEN_DEQ_WO_THRESHOLD 0.50, the carrier's W_x/W_out 0.70).
        Returns the sigma estimates before rescaling, [7][h_slots] (W_q, W_k, W_v, W_o, W_in, W_x,
        W_out)."""
        def thr(name, default, floor):  # env_f32(name).unwrap_or(default).max(floor)
            v = self._env_f32(name)
            return max(default if v is None else v, floor)
        attn = thr("AIDEEN_DEQ_ATTN_THRESHOLD", 0.10, 0.01)
        win = thr("AIDEEN_DEQ_WIN_THRESHOLD", 0.30, 0.05)
        wv = thr("AIDEEN_DEQ_WV_THRESHOLD", 0.50, 0.01)
        wo = thr("AIDEEN_DEQ_WO_THRESHOLD", 0.50, 0.01)
        return self.renormalize_spectral_with(attn, win, 0.70, wv, wo, n_iters)

    def renormalize_spectral_with(self, attn_threshold: float, win_threshold: float, fpm_threshold: float,
                                  wv_threshold: float, wo_threshold: float, n_iters: int = 12) -> np.ndarray:
        """RustDeqBridge::renormalize_spectral (deq_bridge.rs:1742-1791) with explicit thresholds."""
        sig = np.zeros((7, self.model.H), np.float32)
        check(lib().adn_renormalize_spectral(self._ctx, float(attn_threshold), float(win_threshold),
                                             float(fpm_threshold), float(wv_threshold), float(wo_threshold),
                                             int(n_iters), _fp(sig)))
        return sig


class HipBlockBackend:
    """``BlockBackend`` over HIP (the reference's WgpuBlockBackend, gpu_backend.rs:71-248)."""

    def __init__(self, ctx_owner: GpuDeqBackend):
        self._owner = ctx_owner

    def fpm_batch_step(self, x, dt, a, b, c) -> np.ndarray:
        arrs = [np.ascontiguousarray(v, np.float32) for v in (x, dt, a, b, c)]
        d = arrs[0].size
        if any(v.size != d for v in arrs):
            raise _lib.AdnError(_lib.ADN_E_INVALID, "HipBlockBackend: dim mismatch")
        y = np.zeros(d, np.float32)
        check(lib().adn_block_step(self._owner._ctx, d, *[_fp(v) for v in arrs], _fp(y)))
        return y


class HipComputeBackend:
    """``ComputeBackend`` over HIP (the reference's aideen-engine WgpuBackend)."""

    def __init__(self, ctx_owner: GpuDeqBackend):
        self._owner = ctx_owner

    def load_tensor(self, data) -> int:
        a = np.ascontiguousarray(data, np.float32).reshape(-1)
        tid = C.c_int32(0)
        check(lib().adn_load_tensor(self._owner._ctx, _fp(a), a.size, C.byref(tid)))
        return tid.value

    def ffn_forward(self, weights: int, inp: int, out_dim: int) -> np.ndarray:
        y = np.zeros(out_dim, np.float32)
        check(lib().adn_ffn_forward(self._owner._ctx, weights, inp, out_dim, _fp(y)))
        return y
