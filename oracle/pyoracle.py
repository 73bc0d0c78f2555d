"""ctypes binding of the C oracle (TEST INFRASTRUCTURE ONLY).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this module; the
product package never does.  ``build()`` compiles ``liboracle.so`` from ``aideen_oracle.c``.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from typing import Dict, Optional

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

F32P = C.POINTER(C.c_float)
I32P = C.POINTER(C.c_int32)


class OrcCfg(C.Structure):
    _fields_ = [("d", C.c_int32), ("H", C.c_int32), ("V", C.c_int32), ("N", C.c_int32),
                ("r", C.c_int32), ("flags", C.c_uint32), ("max_iters", C.c_int32),
                ("eps", C.c_float), ("beta", C.c_float), ("anderson_m", C.c_int32)]


WEIGHT_FIELDS = ["w_q", "w_k", "w_v", "w_o", "w_in", "q_bias", "k_bias", "anchor", "norm_scale",
                 "embed", "lm_w", "lm_b", "lm_g", "a_log", "wx_diag", "w_out", "b_delta", "w_kw",
                 "w_vw", "w_b", "w_c"]


class OrcWeights(C.Structure):
    _fields_ = [(n, F32P) for n in WEIGHT_FIELDS]


# memory-coupled solve weights (FPMR w_hist_shared, hist_slot_scale, hist_gate_logit)
HIST_FIELDS = [("w_hist", "w_hist"), ("slot_scale", "hist_slot_scale"), ("gate_logit", "hist_gate_logit")]


class OrcHistWeights(C.Structure):
    _fields_ = [(n, F32P) for n, _ in HIST_FIELDS]


def build(quiet: bool = True) -> None:
    subprocess.run(["make", "-s", "-C", HERE], check=True,
                   stdout=subprocess.DEVNULL if quiet else None)


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        L.orc_spectral_norm.restype = C.c_float
        L.orc_spectral_norm.argtypes = [F32P, C.c_int, C.c_int, C.c_int]
        L.orc_normalize.argtypes = [F32P, C.c_int, C.c_int, C.c_float, C.c_int]
        L.orc_normalize_if_needed.argtypes = [F32P, C.c_int, C.c_int, C.c_float, C.c_int]
        L.orc_spectral_norm_gpu.restype = C.c_float
        L.orc_spectral_norm_gpu.argtypes = [F32P, C.c_int, C.c_int]
        L.orc_renorm_gpu.restype = C.c_float
        L.orc_renorm_gpu.argtypes = [F32P, C.c_long, F32P, C.c_int, C.c_float, C.c_int]
        L.orc_damped_update.argtypes = [F32P, F32P, C.c_float, C.c_int, F32P]
        L.orc_signal.argtypes = [C.POINTER(OrcCfg), C.POINTER(OrcWeights), F32P, F32P]
        L.orc_init.argtypes = [C.POINTER(OrcCfg), C.POINTER(OrcWeights), F32P, F32P, F32P]
        L.orc_picard_step.argtypes = [C.POINTER(OrcCfg), C.POINTER(OrcWeights), F32P, F32P, F32P, F32P]
        L.orc_anderson_coeffs.argtypes = [C.c_int, F32P, F32P]
        L.orc_solve_token.restype = C.c_int
        L.orc_solve_token.argtypes = [C.POINTER(OrcCfg), C.POINTER(OrcWeights), F32P, F32P, F32P]
        L.orc_lm_head_token.argtypes = [C.POINTER(OrcCfg), C.POINTER(OrcWeights), F32P, F32P, F32P]
        L.orc_argmax.restype = C.c_int
        L.orc_argmax.argtypes = [F32P, C.c_int]
        L.orc_scan_seq.argtypes = [C.POINTER(OrcCfg), C.POINTER(OrcWeights), C.c_int, F32P, F32P, F32P, F32P]
        L.orc_scan_recirculate.argtypes = [C.POINTER(OrcCfg), C.POINTER(OrcWeights), C.c_int, F32P, F32P, F32P]
        L.orc_forward.argtypes = [C.POINTER(OrcCfg), C.POINTER(OrcWeights), C.c_int, C.c_int, I32P,
                                  F32P, F32P, F32P, I32P, I32P, I32P, F32P, F32P, C.c_int]
        L.orc_model_create.restype = C.c_void_p
        L.orc_model_create.argtypes = [C.POINTER(OrcCfg), C.POINTER(OrcWeights)]
        L.orc_model_forward.argtypes = [C.c_void_p, C.c_int, C.c_int, I32P, F32P, F32P, F32P, I32P,
                                        I32P, I32P, F32P, F32P, C.c_int]
        L.orc_model_free.argtypes = [C.c_void_p]
        L.orc_decode_greedy.argtypes = [C.POINTER(OrcCfg), C.POINTER(OrcWeights), C.POINTER(OrcHistWeights),
                                        C.c_int, C.c_int, I32P, C.c_int, C.c_int, C.c_float, I32P, C.c_int]
        L.orc_decode_sample.argtypes = [C.POINTER(OrcCfg), C.POINTER(OrcWeights), C.POINTER(OrcHistWeights),
                                        C.c_int, C.c_int, I32P, C.c_int, C.c_int, C.c_float, C.c_float, C.c_int,
                                        C.c_float, F32P, I32P, C.POINTER(C.c_double), C.c_int]
        L.orc_lm_sample.restype = C.c_int
        L.orc_lm_sample.argtypes = [F32P, C.c_int, I32P, C.c_int, C.c_float, C.c_float, C.c_int, C.c_float,
                                    C.c_float, C.POINTER(C.c_double)]
        L.orc_hist_ctx.argtypes = [C.POINTER(OrcCfg), C.POINTER(OrcHistWeights), F32P, F32P, F32P]
        L.orc_temporal_step.argtypes = [C.POINTER(OrcCfg), C.POINTER(OrcWeights), F32P, F32P, F32P]
        L.orc_forward_memory.argtypes = [C.POINTER(OrcCfg), C.POINTER(OrcWeights), C.POINTER(OrcHistWeights),
                                         C.c_int, C.c_int, I32P, F32P, F32P, F32P, F32P, I32P, I32P, I32P,
                                         F32P, C.c_int]
        L.orc_zoh_step.argtypes = [C.c_int, F32P, F32P, F32P, F32P, F32P, F32P]
        L.orc_embed_context.argtypes = [C.c_int, F32P, C.c_int, C.c_int, I32P, C.c_int, F32P]
        L.orc_adjoint.argtypes = [C.POINTER(OrcCfg), F32P, C.c_int, F32P, F32P, F32P, C.c_int, C.c_float, F32P, F32P]
        L.orc_gemv_colmajor.argtypes = [F32P, F32P, C.c_int, C.c_int, F32P]
        _lib = L
    return _lib


def fp(a: Optional[np.ndarray]):
    if a is None:
        return None
    assert a.dtype == np.float32 and a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(F32P)


def ip(a: Optional[np.ndarray]):
    if a is None:
        return None
    assert a.dtype == np.int32 and a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(I32P)


class Oracle:
    """Holds one model (config + weights) for repeated oracle calls."""

    def __init__(self, cfg, weights: Dict[str, Optional[np.ndarray]]):
        self.mc = cfg
        self.c = OrcCfg(cfg.d, cfg.H, cfg.V, cfg.N, cfg.r, cfg.flags, cfg.max_iters,
                        cfg.eps, cfg.beta, cfg.anderson_m)
        self._keep = {k: (None if v is None else np.ascontiguousarray(v, dtype=np.float32))
                      for k, v in weights.items()}
        self.w = OrcWeights(**{k: fp(self._keep.get(k)) for k in WEIGHT_FIELDS})
        self.hw = OrcHistWeights(**{n: fp(self._keep.get(k)) for n, k in HIST_FIELDS})
        self.L = lib()

    # --- per-token pieces -------------------------------------------------
    def signal(self, x):
        out = np.zeros((self.mc.H, self.mc.d), np.float32)
        self.L.orc_signal(C.byref(self.c), C.byref(self.w), fp(np.ascontiguousarray(x, np.float32)), fp(out))
        return out

    def init(self, x, signal):
        out = np.zeros((self.mc.H, self.mc.d), np.float32)
        self.L.orc_init(C.byref(self.c), C.byref(self.w), fp(np.ascontiguousarray(x, np.float32)),
                        fp(np.ascontiguousarray(signal, np.float32)), fp(out))
        return out

    def step(self, h, signal):
        out = np.zeros((self.mc.H, self.mc.d), np.float32)
        attn = np.zeros((self.mc.H, self.mc.H), np.float32)
        self.L.orc_picard_step(C.byref(self.c), C.byref(self.w), fp(np.ascontiguousarray(h, np.float32)),
                               fp(np.ascontiguousarray(signal, np.float32)), fp(out), fp(attn))
        return out, attn

    def solve(self, x):
        h = np.zeros((self.mc.H, self.mc.d), np.float32)
        trace = np.zeros(max(self.mc.max_iters, 1), np.float32)
        it = self.L.orc_solve_token(C.byref(self.c), C.byref(self.w),
                                    fp(np.ascontiguousarray(x, np.float32)), fp(h), fp(trace))
        return h, it, trace[:it]

    def lm_head(self, h_star):
        pooled = np.zeros(self.mc.d, np.float32)
        logits = np.zeros(self.mc.V, np.float32)
        self.L.orc_lm_head_token(C.byref(self.c), C.byref(self.w),
                                 fp(np.ascontiguousarray(h_star, np.float32)), fp(pooled), fp(logits))
        return pooled, logits

    def scan(self, h_star_seq, state_in=None):
        T = h_star_seq.shape[0]
        y = np.zeros((T, self.mc.H, self.mc.d), np.float32)
        st = np.zeros((self.mc.H, self.mc.d, self.mc.N), np.float32)
        self.L.orc_scan_seq(C.byref(self.c), C.byref(self.w), T,
                            fp(np.ascontiguousarray(h_star_seq, np.float32)),
                            fp(None if state_in is None else np.ascontiguousarray(state_in, np.float32)),
                            fp(y), fp(st))
        return y, st

    def scan_recirculate(self, h_star_seq, m_in=None):
        T = h_star_seq.shape[0]
        y = np.zeros((T, self.mc.H, self.mc.d), np.float32)
        self.L.orc_scan_recirculate(C.byref(self.c), C.byref(self.w), T,
                                    fp(np.ascontiguousarray(h_star_seq, np.float32)),
                                    fp(None if m_in is None else np.ascontiguousarray(m_in, np.float32)),
                                    fp(y))
        return y

    # --- clean adjoint ----------------------------------------------------------
    def adjoint(self, signal, h_star, dl, iters, beta=None):
        """signal, h_star [ntok][H][d], dl [ntok][d] -> (v [ntok][H][d], source grad [ntok][d])."""
        signal = np.ascontiguousarray(signal, np.float32).reshape(-1, self.mc.H, self.mc.d)
        ntok = signal.shape[0]
        v = np.zeros((ntok, self.mc.H, self.mc.d), np.float32)
        src = np.zeros((ntok, self.mc.d), np.float32)
        self.L.orc_adjoint(C.byref(self.c), fp(self._keep["norm_scale"]), ntok, fp(signal),
                           fp(np.ascontiguousarray(h_star, np.float32)), fp(np.ascontiguousarray(dl, np.float32)),
                           iters, self.mc.beta if beta is None else beta, fp(v), fp(src))
        return v, src

    # --- memory-coupled solve ------------------------------------------------
    def hist_ctx(self, m_prev, signal):
        out = np.zeros((self.mc.H, self.mc.d), np.float32)
        self.L.orc_hist_ctx(C.byref(self.c), C.byref(self.hw),
                            fp(None if m_prev is None else np.ascontiguousarray(m_prev, np.float32)),
                            fp(np.ascontiguousarray(signal, np.float32)), fp(out))
        return out

    def temporal_step(self, m_prev, h_star):
        out = np.zeros((self.mc.H, self.mc.d), np.float32)
        self.L.orc_temporal_step(C.byref(self.c), C.byref(self.w),
                                 fp(None if m_prev is None else np.ascontiguousarray(m_prev, np.float32)),
                                 fp(np.ascontiguousarray(h_star, np.float32)), fp(out))
        return out

    def forward_memory(self, tokens, m_in=None, nthreads=0):
        """Memory-coupled forward; returns h_star, pooled, logits, argmax, iters and m_seq (every
        carrier state m_t)."""
        tokens = np.ascontiguousarray(tokens, dtype=np.int32)
        B, T = tokens.shape
        mc = self.mc
        out = dict(h_star=np.zeros((B, T, mc.H, mc.d), np.float32),
                   pooled=np.zeros((B, T, mc.d), np.float32),
                   logits=np.zeros((B, T, mc.V), np.float32),
                   iters=np.zeros((B, T), np.int32), converged=np.zeros((B, T), np.int32),
                   argmax=np.zeros((B, T), np.int32), m_seq=np.zeros((B, T, mc.H, mc.d), np.float32))
        self.L.orc_forward_memory(C.byref(self.c), C.byref(self.w), C.byref(self.hw), B, T, ip(tokens),
                                  fp(None if m_in is None else np.ascontiguousarray(m_in, np.float32)),
                                  fp(out["h_star"]), fp(out["pooled"]), fp(out["logits"]),
                                  ip(out["iters"]), ip(out["converged"]), ip(out["argmax"]), fp(out["m_seq"]),
                                  nthreads)
        return out

    # --- whole forward ------------------------------------------------------
    def forward(self, tokens, want_logits=True, want_scan=True, nthreads=0):
        tokens = np.ascontiguousarray(tokens, dtype=np.int32)
        B, T = tokens.shape
        mc = self.mc
        out = dict(
            h_star=np.zeros((B, T, mc.H, mc.d), np.float32),
            pooled=np.zeros((B, T, mc.d), np.float32),
            iters=np.zeros((B, T), np.int32),
            converged=np.zeros((B, T), np.int32),
            argmax=np.zeros((B, T), np.int32),
        )
        if want_logits:
            out["logits"] = np.zeros((B, T, mc.V), np.float32)
        if want_scan:
            out["scan_y"] = np.zeros((B, T, mc.H, mc.d), np.float32)
            out["scan_state"] = np.zeros((B, mc.H, mc.d, mc.N), np.float32)
        self.L.orc_forward(C.byref(self.c), C.byref(self.w), B, T, ip(tokens),
                           fp(out["h_star"]), fp(out["pooled"]), fp(out.get("logits")),
                           ip(out["iters"]), ip(out["converged"]), ip(out["argmax"]), fp(out.get("scan_y")),
                           fp(out.get("scan_state")), nthreads)
        return out

    def prepared(self):
        """A model handle with the CPU-side weight layout done once (for timing)."""
        return _Prepared(self)

    def decode_greedy(self, prompt, n_new, ctx_len, rep_penalty=1.0, nthreads=0):
        """Trainer::generate's greedy loop: prompt [B][T0] -> the n_new appended tokens [B][n_new]
        (the model config's max_iters / eps / beta drive each solve; generate uses 10, 0)."""
        prompt = np.ascontiguousarray(prompt, dtype=np.int32)
        B, T0 = prompt.shape
        out = np.zeros((B, n_new), np.int32)
        self.L.orc_decode_greedy(C.byref(self.c), C.byref(self.w), C.byref(self.hw), B, T0, ip(prompt),
                                 n_new, ctx_len, rep_penalty, ip(out), nthreads)
        return out


    def decode_sample(self, prompt, n_new, ctx_len, temperature, top_p, top_k, rep_penalty, uniforms,
                      nthreads=0):
        """The same loop with LmHead::sample: uniforms [B][n_new] the draws -> (tokens [B][n_new],
        each step's conditioning [B][n_new], >= 1 where rounding cannot change the draw)."""
        prompt = np.ascontiguousarray(prompt, dtype=np.int32)
        B, T0 = prompt.shape
        uni = np.ascontiguousarray(uniforms, np.float32).reshape(B, n_new)
        out = np.zeros((B, n_new), np.int32)
        cond = np.zeros((B, n_new), np.float64)
        self.L.orc_decode_sample(C.byref(self.c), C.byref(self.w), C.byref(self.hw), B, T0, ip(prompt), n_new,
                                 ctx_len, float(temperature), float(top_p), int(top_k), float(rep_penalty),
                                 fp(uni), ip(out), cond.ctypes.data_as(C.POINTER(C.c_double)), nthreads)
        return out, cond


class _Prepared:
    def __init__(self, o: "Oracle"):
        self.o = o
        self.h = o.L.orc_model_create(C.byref(o.c), C.byref(o.w))

    def forward(self, tokens, nthreads=0, want_logits=True, want_scan=True):
        """Same outputs as Oracle.forward (logits/scan optional); returns the output dict."""
        o, mc = self.o, self.o.mc
        tokens = np.ascontiguousarray(tokens, dtype=np.int32)
        B, T = tokens.shape
        out = dict(h_star=np.zeros((B, T, mc.H, mc.d), np.float32), iters=np.zeros((B, T), np.int32),
                   argmax=np.zeros((B, T), np.int32))
        if want_logits:
            out["logits"] = np.zeros((B, T, mc.V), np.float32)
        if want_scan:
            out["scan_y"] = np.zeros((B, T, mc.H, mc.d), np.float32)
            out["scan_state"] = np.zeros((B, mc.H, mc.d, mc.N), np.float32)
        o.L.orc_model_forward(self.h, B, T, ip(tokens), fp(out["h_star"]), None, fp(out.get("logits")),
                              ip(out["iters"]), None, ip(out["argmax"]), fp(out.get("scan_y")),
                              fp(out.get("scan_state")), nthreads)
        return out

    def __del__(self):
        try:
            self.o.L.orc_model_free(self.h)
        except Exception:
            pass


def spectral_norm(w: np.ndarray, n_iter: int = 20) -> float:
    w = np.ascontiguousarray(w, np.float32)
    return lib().orc_spectral_norm(fp(w), w.shape[0], w.shape[1], n_iter)


def normalize(w: np.ndarray, target: float, n_iter: int = 20) -> np.ndarray:
    w = np.ascontiguousarray(w, np.float32).copy()
    lib().orc_normalize(fp(w), w.shape[0], w.shape[1], target, n_iter)
    return w


def normalize_if_needed(w: np.ndarray, threshold: float, n_iter: int = 20) -> np.ndarray:
    w = np.ascontiguousarray(w, np.float32).copy()
    lib().orc_normalize_if_needed(fp(w), w.shape[0], w.shape[1], threshold, n_iter)
    return w


def spectral_norm_gpu(wg: np.ndarray, n_iters: int = 12) -> float:
    """spectral_renorm.wgsl's sigma estimate of the d x d buffer wg (indexed wg[i, j])."""
    wg = np.ascontiguousarray(wg, np.float32)
    return lib().orc_spectral_norm_gpu(fp(wg), wg.shape[0], n_iters)


# (weight, threshold index, buffer form) of renormalize_spectral's roles: the reference's buffers
# are [in][out] per slot for W_q/W_k/W_v/W_o (w_*_gpu_flat, fixed_point_memory_reasoning.rs:516-561)
# and for the carrier's W_out (nalgebra's column-major storage), the CPU matrix for W_in (uploaded
# row-major, read transposed by the forward kernel: D2), and the diagonal for W_x (what the carrier
# keeps of it).  Thresholds: (attn, win, fpm, wv, wo).
RENORM_ROLES = (("w_q", 0, "T"), ("w_k", 0, "T"), ("w_v", 3, "T"), ("w_o", 4, "T"), ("w_in", 1, "N"),
                ("wx_diag", 2, "diag"), ("w_out", 2, "T"))


def renormalize_spectral(weights: Dict[str, Optional[np.ndarray]], thresholds=(0.10, 0.30, 0.70, 0.50, 0.50),
                         n_iters: int = 12):
    """GpuDeqBackend::renormalize_spectral (gpu_deq.rs:5567-5591; deq_bridge.rs:1742-1791;
    spectral_renorm.wgsl:83-196) on a weight dict in include/aideen_hip.h's [s][out][in] layout:
    (renormalised copy, sigmas [7][H] in RENORM_ROLES order, 0 for an absent W_out)."""
    w = {k: (None if v is None else np.array(v, np.float32, copy=True)) for k, v in weights.items()}
    H = w["w_q"].shape[0]
    sig = np.zeros((7, H), np.float32)
    for role, (name, ti, form) in enumerate(RENORM_ROLES):
        if w.get(name) is None:
            continue
        for s in range(H):
            m = np.ascontiguousarray(w[name][s])
            if form == "T":
                wg = np.ascontiguousarray(m.T)
            elif form == "N":
                wg = m
            else:
                wg = np.diag(m).astype(np.float32)
            sig[role, s] = lib().orc_renorm_gpu(fp(m), m.size, fp(wg), wg.shape[0], float(thresholds[ti]), n_iters)
            w[name][s] = m
    return w, sig


def damped_update(h, f, beta):
    h = np.ascontiguousarray(h, np.float32)
    f = np.ascontiguousarray(f, np.float32)
    out = np.zeros_like(h)
    lib().orc_damped_update(fp(h), fp(f), beta, h.size, fp(out))
    return out


def anderson_coeffs(g: np.ndarray) -> np.ndarray:
    g = np.ascontiguousarray(g, np.float32)
    beta = np.zeros(g.shape[0], np.float32)
    lib().orc_anderson_coeffs(g.shape[0], fp(g), fp(beta))
    return beta


def argmax(logits: np.ndarray) -> int:
    logits = np.ascontiguousarray(logits, np.float32)
    return lib().orc_argmax(fp(logits), logits.size)


def lm_sample(logits, context, temperature: float, top_p: float, top_k: int, rep_penalty: float, r: float):
    """LmHead::sample (lm_head.rs:78-168) with the draw r given: (token, conditioning, length of
    the kept list)."""
    logits = np.ascontiguousarray(logits, np.float32)
    ctx = np.ascontiguousarray(context if context is not None else [], np.int32)
    cond = (C.c_double * 2)()
    t = lib().orc_lm_sample(fp(logits), logits.size, ip(ctx), ctx.size, float(temperature), float(top_p),
                            int(top_k), float(rep_penalty), float(r), cond)
    return t, cond[0], int(cond[1])


def zoh_step(x, dt, a, b, c):
    arrs = [np.ascontiguousarray(v, np.float32) for v in (x, dt, a, b, c)]
    y = np.zeros_like(arrs[0])
    lib().orc_zoh_step(arrs[0].size, *[fp(v) for v in arrs], fp(y))
    return y


def gemv_colmajor(w, x, out_dim):
    w = np.ascontiguousarray(w, np.float32)
    x = np.ascontiguousarray(x, np.float32)
    y = np.zeros(out_dim, np.float32)
    lib().orc_gemv_colmajor(fp(w), fp(x), x.size, out_dim, fp(y))
    return y


def embed_context(embed: np.ndarray, tokens: np.ndarray, ctx: int) -> np.ndarray:
    """tokenizer.rs:133-149 embed_context for the window ending at every position of every
    sequence; tokens [B][T] -> [B][T][d]."""
    embed = np.ascontiguousarray(embed, np.float32)
    tokens = np.ascontiguousarray(tokens, np.int32)
    B, T = tokens.shape
    d = embed.shape[1]
    out = np.zeros((B, T, d), np.float32)
    lib().orc_embed_context(d, fp(embed), B, T, ip(tokens), ctx, fp(out))
    return out
