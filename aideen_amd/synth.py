"""Deterministic synthetic model weights and token streams.

The reference seeds its weights with rand 0.8.5's ChaCha12 ``StdRng``
(``aideen-backbone/src/fixed_point_memory_reasoning.rs:244-247``), a stream that cannot be
reproduced without Rust.  This module defines the build's own generator: a counter-based
SplitMix64 stream per named tensor, so every tensor is a pure function of (seed, name, shape).
Parity is therefore taken oracle-vs-GPU on identical tensors.

What follows the reference exactly:

* Xavier-uniform range ``sqrt(3/d)`` (FPMR:259-260) and the spectral rescale by power
  iteration from ``u0 = 1/sqrt(rows)`` (``spectral_norm.rs:25-71``);
* the embedding closed form ``((i*d+j) as f32 * 1.6180339) % 1.0 - 0.5) * 0.5/sqrt(d)``
  (``tokenizer.rs:62-66``) and the LM-head closed form with scale ``0.1/sqrt(d)``
  (``lm_head.rs:21-33``), in f32 arithmetic;
* the a_log prior ``logit(0.80 + alpha*(0.999-0.80))`` across slots (FPMR:367-381), the
  ``U(-0.01, 0.01)`` W_x / W_out / write-path inits (FPMR:276-290) and ``b_delta = 0``.

Transcendental init values are evaluated in float64 and rounded once to float32, and the
spectral scale factor is rounded to float32, so the tensors do not depend on the host's SIMD
math library.
"""
from __future__ import annotations

import dataclasses
import hashlib
from typing import Dict, Optional

import numpy as np

F_WIN_TRANSPOSED = 1 << 0
F_SCORE_CLAMP4 = 1 << 1
F_RMS_EXCL_ANCHOR = 1 << 2
F_INIT_SIGNAL_RMS = 1 << 3
F_RESID_L2 = 1 << 4
F_SCAN_SELECTIVE = 1 << 5
F_GEMM_FP32 = 1 << 6
F_GEMM_BF16X3 = 1 << 7
F_GEMM_BF16 = 1 << 8
F_MEMORY = 1 << 9
F_TOKEN_CARRY = 1 << 10
F_RESID_RELRMS = 1 << 11
F_HOMEOSTATIC_EXIT = 1 << 12

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def _fnv1a64(text: str) -> int:
    h = 0xCBF29CE484222325
    for b in text.encode():
        h ^= b
        h = (h * 0x100000001B3) & 0xFFFFFFFFFFFFFFFF
    return h


def splitmix64(seed: int, n: int, offset: int = 0) -> np.ndarray:
    """Outputs ``offset .. offset+n-1`` of the SplitMix64 stream started at ``seed``."""
    with np.errstate(over="ignore"):
        idx = np.arange(offset + 1, offset + n + 1, dtype=np.uint64)
        z = np.uint64(seed) + idx * _GOLDEN
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


def _stream_seed(seed: int, name: str) -> int:
    return int(splitmix64(seed ^ _fnv1a64(name), 1)[0])


def uniform(seed: int, name: str, shape, lo: float, hi: float) -> np.ndarray:
    """U[lo, hi) in float32: lo + (hi-lo) * (z >> 40) * 2^-24."""
    n = int(np.prod(shape))
    z = splitmix64(_stream_seed(seed, name), n)
    u = (z >> np.uint64(40)).astype(np.float32) * np.float32(2.0 ** -24)
    return (np.float32(lo) + np.float32(hi - lo) * u).astype(np.float32).reshape(shape)


def normal(seed: int, name: str, shape) -> np.ndarray:
    """N(0,1) by Box-Muller on two uniform streams, evaluated in float64."""
    n = int(np.prod(shape))
    z1 = splitmix64(_stream_seed(seed, name + "#a"), n)
    z2 = splitmix64(_stream_seed(seed, name + "#b"), n)
    u1 = ((z1 >> np.uint64(11)).astype(np.float64) + 1.0) * 2.0 ** -53
    u2 = (z2 >> np.uint64(11)).astype(np.float64) * 2.0 ** -53
    g = np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)
    return g.astype(np.float32).reshape(shape)


def spectral_norm_f64(w: np.ndarray, n_iter: int = 20) -> float:
    """spectral_norm.rs:25-59 power iteration (u0 = 1/sqrt(rows)), in float64."""
    w64 = w.astype(np.float64)
    rows, cols = w64.shape
    u = np.full(rows, 1.0 / np.sqrt(rows))
    sigma = 1.0
    for _ in range(n_iter):
        v = w64.T @ u
        nv = np.linalg.norm(v)
        if nv < 1e-12:
            return 0.0
        v /= nv
        wv = w64 @ v
        nu = np.linalg.norm(wv)
        if nu < 1e-12:
            return 0.0
        u = wv / nu
        sigma = float(u @ (w64 @ v))
    return max(abs(sigma), 1e-12)


def rescale_to(w: np.ndarray, target: float, n_iter: int = 20) -> np.ndarray:
    """spectral_norm.rs:65-71 normalize(): W * (target / sigma), scale rounded to f32."""
    sigma = spectral_norm_f64(w, n_iter)
    if sigma < 1e-12:
        return w.copy()
    return (w * np.float32(target / sigma)).astype(np.float32)


def golden_ratio_table(rows: int, d: int, scale_mult: float) -> np.ndarray:
    """tokenizer.rs:62-66 / lm_head.rs:24-29 closed form in f32 arithmetic."""
    idx = np.arange(rows * d, dtype=np.int64).astype(np.float32)
    v = np.fmod(idx * np.float32(1.6180339), np.float32(1.0))
    scale = (np.float32(1.0) / np.sqrt(np.float32(d))) * np.float32(scale_mult)
    return ((v - np.float32(0.5)) * scale).astype(np.float32).reshape(rows, d)


def zipf_tokens(seed: int, name: str, n: int, vocab: int, s: float = 1.1) -> np.ndarray:
    """Zipf(s) ranks over [0, vocab) by inverse CDF; rank k -> token id k."""
    w = 1.0 / np.arange(1, vocab + 1, dtype=np.float64) ** s
    cdf = np.cumsum(w)
    cdf /= cdf[-1]
    z = splitmix64(_stream_seed(seed, name), n)
    u = (z >> np.uint64(11)).astype(np.float64) * 2.0 ** -53
    return np.minimum(np.searchsorted(cdf, u, side="right"), vocab - 1).astype(np.int32)


def uniform_tokens(seed: int, name: str, n: int, vocab: int) -> np.ndarray:
    z = splitmix64(_stream_seed(seed, name), n)
    return (z % np.uint64(vocab)).astype(np.int32)


@dataclasses.dataclass
class ModelConfig:
    d: int
    H: int
    V: int
    N: int = 1
    r: int = 32
    flags: int = F_SCAN_SELECTIVE
    max_iters: int = 20
    eps: float = 1e-4
    beta: float = 0.70
    anderson_m: int = 0
    sigma: float = 0.5            # spectral norm of each block matrix
    win_sigma: Optional[float] = None  # defaults to sigma
    qk_bias: bool = False

    def as_dict(self) -> dict:
        return dataclasses.asdict(self)


# BASELINE.json configs.  C1 = the reference's CPU-runnable plumbing case (golden fixtures);
# NS = the north-star throughput case (bench workload).
PRESETS = {
    "C1": dict(model=ModelConfig(d=128, H=4, V=512, N=16), B=1, T=64, tokens="uniform"),
    "C2": dict(model=ModelConfig(d=512, H=8, V=50257, N=16), B=1, T=256, tokens="zipf"),
    "NS": dict(model=ModelConfig(d=512, H=8, V=50257, N=16), B=32, T=256, tokens="zipf"),
    "C3": dict(model=ModelConfig(d=512, H=8, V=50257, N=16, sigma=0.7, anderson_m=5),
               B=32, T=1024, tokens="zipf"),
    # long-context scan stress: input-dependent decay logits N(0,1) through the model's own
    # projection, decay bases spread from ~0.999 to ~0.01 across channels (make_weights)
    "C4": dict(model=ModelConfig(d=512, H=8, V=50257, N=16), B=8, T=8192, tokens="uniform",
               long_memory_gates=True),
    "C5": dict(model=ModelConfig(d=2048, H=16, V=50257, N=32, sigma=0.8, anderson_m=5),
               B=16, T=2048, tokens="zipf"),
}


def preset_weights(name: str, cfg: Optional[ModelConfig] = None, seed: int = 0) -> Dict[str, Optional[np.ndarray]]:
    """The weights of a BASELINE preset (cfg overrides its model, e.g. with other GEMM flags)."""
    p = PRESETS[name]
    return make_weights(cfg or p["model"], seed=seed, long_memory_gates=p.get("long_memory_gates", False))


def make_weights(cfg: ModelConfig, seed: int = 0, gates_seed: int = 2,
                 long_memory_gates: bool = False) -> Dict[str, Optional[np.ndarray]]:
    """All tensors of one model, in the layouts of include/aideen_hip.h (W[s][out][in])."""
    d, H, V, N, r = cfg.d, cfg.H, cfg.V, cfg.N, cfg.r
    xr = float(np.sqrt(np.float32(3.0) / np.float32(d)))
    w: Dict[str, Optional[np.ndarray]] = {}
    for name in ("w_q", "w_k", "w_v", "w_o", "w_in"):
        target = cfg.sigma if name != "w_in" or cfg.win_sigma is None else cfg.win_sigma
        mats = uniform(seed, name, (H, d, d), -xr, xr)
        w[name] = np.stack([rescale_to(mats[s], target) for s in range(H)])
    if cfg.qk_bias:
        w["q_bias"] = uniform(seed, "q_bias", (H, d), -0.08, 0.08)
        w["k_bias"] = uniform(seed, "k_bias", (H, d), -0.08, 0.08)
    else:
        w["q_bias"] = None
        w["k_bias"] = None
    w["anchor"] = uniform(seed, "anchor", (H, d), -1.0, 1.0)
    w["norm_scale"] = np.ones(d, dtype=np.float32)
    w["embed"] = golden_ratio_table(V, d, 0.5)
    w["lm_w"] = golden_ratio_table(V, d, 0.1)
    w["lm_b"] = np.zeros(V, dtype=np.float32)
    w["lm_g"] = np.ones(d, dtype=np.float32)
    # FPMR:367-381: a in [0.80, 0.999] across slots, stored as logit(a).
    alpha = np.full(H, 0.5) if H <= 1 else np.arange(H, dtype=np.float64) / (H - 1)
    a = 0.80 + alpha * (0.999 - 0.80)
    a_log = np.repeat(np.log(a / (1.0 - a))[:, None], d, axis=1)
    if long_memory_gates:
        # C4: decay bases spread from ~0.999 (long memory) to ~0.01 across channels, and
        # input-dependent gate logits drawn N(0,1) through the model's own projection.
        frac = (np.arange(H * d, dtype=np.float64).reshape(H, d) % d) / max(d - 1, 1)
        base = 0.999 + frac * (0.01 - 0.999)
        a_log = np.log((1.0 - base) / base)
    w["a_log"] = a_log.astype(np.float32)
    w["wx_diag"] = uniform(seed, "w_x", (H, d), -0.01, 0.01)
    w["w_out"] = uniform(seed, "w_out", (H, d, d), -0.01, 0.01)
    if long_memory_gates:
        w["b_delta"] = normal(gates_seed, "b_delta", (H, d))
        w["w_kw"] = (normal(gates_seed, "w_kw", (H, d, r)) / np.float32(np.sqrt(d))).astype(np.float32)
        w["w_vw"] = (normal(gates_seed, "w_vw", (H, r, d)) / np.float32(np.sqrt(r))).astype(np.float32)
    else:
        w["b_delta"] = np.zeros((H, d), dtype=np.float32)
        w["w_kw"] = uniform(seed, "w_kw", (H, d, r), -0.01, 0.01)
        w["w_vw"] = uniform(seed, "w_vw", (H, r, d), -0.01, 0.01)
    if N > 1:
        w["w_b"] = uniform(seed, "w_b", (H, N, d), -xr, xr)
        w["w_c"] = uniform(seed, "w_c", (H, N, d), -xr, xr)
    else:
        w["w_b"] = None
        w["w_c"] = None
    return w


def make_token_sensitive_weights(cfg: ModelConfig, seed: int = 0,
                                 long_memory_gates: bool = False) -> Dict[str, Optional[np.ndarray]]:
    """A weight set whose outputs depend strongly on the token, for parity tests that must be able
    to fail on a per-token error (a row written to the wrong token, a shifted index).

    With the reference's own initialisation the solve is anchor-dominated: the anchors are U(-1, 1)
    (FPMR:225-232) while an embedding row of the golden-ratio closed form has entries below
    0.25/sqrt(d), and the closed forms of E and W_lm (f32 index cast) repeat rows.  Here, on top of
    ``make_weights``: anchors x0.02, W_in at spectral norm 3, seeded random E = U(+-0.2) (every
    row distinct), W_lm at Xavier range sqrt(3/d), a random bias U(+-0.05) and an LM-head gain
    U(0.75, 1.25).  The signal W_in x then dominates the anchor, so the solve
    is token-driven and still contracts (NS shape: 10-12 Picard iterations, the logits' token-
    dependent part of order 1, as many distinct arg-max values as distinct tokens)."""
    w = make_weights(dataclasses.replace(cfg, win_sigma=3.0), seed=seed, long_memory_gates=long_memory_gates)
    d, V = cfg.d, cfg.V
    xr = float(np.sqrt(np.float32(3.0) / np.float32(d)))
    w["anchor"] = (w["anchor"] * np.float32(0.02)).astype(np.float32)
    w["embed"] = uniform(seed, "ts_embed", (V, d), -0.2, 0.2)
    w["lm_w"] = uniform(seed, "ts_lm_w", (V, d), -xr, xr)
    w["lm_b"] = uniform(seed, "ts_lm_b", (V,), -0.05, 0.05)
    w["lm_g"] = uniform(seed, "ts_lm_g", (d,), 0.75, 1.25)
    return w


WEIGHT_SETS = ("preset", "token_sensitive")


def weights_of_kind(kind: str, cfg: ModelConfig, seed: int = 0,
                    long_memory_gates: bool = False) -> Dict[str, Optional[np.ndarray]]:
    """``make_weights`` ("preset": the reference's initialisation) or
    ``make_token_sensitive_weights`` ("token_sensitive")."""
    if kind == "preset":
        return make_weights(cfg, seed=seed, long_memory_gates=long_memory_gates)
    if kind == "token_sensitive":
        return make_token_sensitive_weights(cfg, seed=seed, long_memory_gates=long_memory_gates)
    raise ValueError(f"unknown weight set {kind!r}")


def make_hist_weights(cfg: ModelConfig, seed: int = 0, strong: bool = False) -> Dict[str, np.ndarray]:
    """Weights of the memory-coupled solve, following the reference's initial values
    (FPMR:279 w_hist_shared = 0.15 I + U(+-0.01); FPMR:312-318 hist_slot_scale = centred slot *
    5e-5 + U(+-1e-4); FPMR:327-333 hist_gate_logit = -1.204 + centred slot * 0.02).  ``strong``
    widens hist_slot_scale to U(+-0.5) and the gate logits to U(-2, 2) so that every term of
    the history context matters in tests.  Kept apart from make_weights so that the digests of
    existing fixtures do not change."""
    d, H = cfg.d, cfg.H
    centred = (np.arange(H, dtype=np.float32) - np.float32((H - 1) * 0.5))[:, None]
    w_hist = (np.eye(d, dtype=np.float32) * np.float32(0.15)
              + uniform(seed, "w_hist_shared", (d, d), -0.01, 0.01))
    if strong:
        scale = uniform(seed, "hist_slot_scale", (H, d), -0.5, 0.5)
        gate = uniform(seed, "hist_gate_logit", (H,), -2.0, 2.0)
    else:
        scale = centred * np.float32(5e-5) + uniform(seed, "hist_slot_scale", (H, d), -1e-4, 1e-4)
        gate = (np.float32(-1.204) + centred[:, 0] * np.float32(0.02)).astype(np.float32)
    return {"w_hist": w_hist.astype(np.float32), "hist_slot_scale": scale.astype(np.float32),
            "hist_gate_logit": gate.astype(np.float32)}


def make_tokens(kind: str, B: int, T: int, vocab: int, seed: int = 1) -> np.ndarray:
    if kind == "zipf":
        return zipf_tokens(seed, "tokens", B * T, vocab).reshape(B, T)
    return uniform_tokens(seed, "tokens", B * T, vocab).reshape(B, T)


def weights_digest(w: Dict[str, Optional[np.ndarray]]) -> str:
    h = hashlib.sha256()
    for k in sorted(w):
        h.update(k.encode())
        if w[k] is not None:
            h.update(np.ascontiguousarray(w[k]).tobytes())
    return h.hexdigest()
