"""`.aidn` checkpoints (``AidenModel``, aideen-core/src/model.rs:10-58).

The reference serialises ``AidenModel { config, weights, metadata }`` with bincode 1.3 (default
options): little-endian fixed-width integers (``usize`` as u64), a u64 length before every string
and sequence, ``bool`` as one byte, struct fields in declaration order, maps as a u64 entry count
followed by key/value pairs.  ``ArchitectureConfig`` is declared in aideen-core/src/state.rs:7-35.

This module holds:
- ``encode`` / ``decode`` (and ``write_aidn`` / ``read_aidn``): the format in Python, used to make
  checkpoints for tests and to cross-check the library's loader;
- ``reference_export``: a model whose slots share their matrices, written under the reference's
  names and layouts (FixedPointMemoryReasoning::export_weights,
  fixed_point_memory_reasoning.rs:626-784; LmHead::export_weights, lm_head.rs:169-188;
  Trainer::save_full, trainer.rs:6472-6530);
- ``AidnModel``: the library's C++ loader (``adn_aidn_*``) through the C ABI.
"""
from __future__ import annotations

import ctypes as C
import struct
from typing import Dict, Optional, Tuple

import numpy as np

# (field, struct code) in declaration order, state.rs:7-35
CONFIG_FIELDS = [
    ("d_m", "Q"), ("d_r", "Q"), ("d_c", "Q"), ("d_e", "Q"), ("d_sim", "Q"), ("h_slots", "Q"),
    ("vocab_size", "Q"), ("ctx_len", "Q"), ("max_deq_iters", "Q"), ("deq_epsilon", "f"),
    ("adj_iters", "Q"), ("train_deq", "?"), ("deq_grad_scale", "f"), ("renorm_every_steps", "Q"),
    ("num_samples", "Q"), ("weight_decay", "f"),
]
# ArchitectureConfig::default (state.rs:37-57)
DEFAULT_CONFIG = dict(d_m=1024, d_r=512, d_c=256, d_e=256, d_sim=1024, h_slots=8, vocab_size=50257,
                      ctx_len=512, max_deq_iters=16, deq_epsilon=1e-4, adj_iters=2, train_deq=True,
                      deq_grad_scale=1.0, renorm_every_steps=4, num_samples=512, weight_decay=0.01)
RETAIN_RANK = 32  # fixed_point_memory_reasoning.rs:291


def _str(s: str) -> bytes:
    b = s.encode("utf-8")
    return struct.pack("<Q", len(b)) + b


def encode(config: dict, weights: Dict[str, np.ndarray], metadata: Dict[str, str]) -> bytes:
    cfg = dict(DEFAULT_CONFIG)
    cfg.update(config)
    out = [b"".join(struct.pack("<" + code, cfg[name]) for name, code in CONFIG_FIELDS)]
    out.append(struct.pack("<Q", len(weights)))
    for name, v in weights.items():
        a = np.ascontiguousarray(v, dtype="<f4").reshape(-1)
        out.append(_str(name) + struct.pack("<Q", a.size) + a.tobytes())
    out.append(struct.pack("<Q", len(metadata)))
    for k, v in metadata.items():
        out.append(_str(k) + _str(v))
    return b"".join(out)


def decode(data: bytes) -> Tuple[dict, Dict[str, np.ndarray], Dict[str, str]]:
    pos = 0

    def take(fmt: str):
        nonlocal pos
        n = struct.calcsize(fmt)
        if pos + n > len(data):
            raise ValueError("truncated .aidn data")
        v = struct.unpack_from(fmt, data, pos)
        pos += n
        return v[0]

    def string() -> str:
        nonlocal pos
        n = take("<Q")
        if pos + n > len(data):
            raise ValueError("truncated .aidn data")
        s = data[pos:pos + n].decode("utf-8")
        pos += n
        return s

    config = {name: take("<" + code) for name, code in CONFIG_FIELDS}
    weights = {}
    for _ in range(take("<Q")):
        name = string()
        n = take("<Q")
        if pos + 4 * n > len(data):
            raise ValueError("truncated .aidn data")
        weights[name] = np.frombuffer(data, dtype="<f4", count=n, offset=pos).astype(np.float32)
        pos += 4 * n
    metadata = {}
    for _ in range(take("<Q")):
        k = string()
        metadata[k] = string()
    if pos != len(data):
        raise ValueError("trailing bytes after the model")
    return config, weights, metadata


def write_aidn(path: str, config: dict, weights: Dict[str, np.ndarray], metadata: Dict[str, str]) -> None:
    with open(path, "wb") as f:
        f.write(encode(config, weights, metadata))


def read_aidn(path: str):
    with open(path, "rb") as f:
        return decode(f.read())


def reference_export(mc, w: Dict[str, Optional[np.ndarray]], damping: float = 0.70,
                     w_x_offdiag: Optional[np.ndarray] = None):
    """A model whose slots share w_q, w_k, w_v, w_o, w_in, w_out, wx_diag and b_delta (slot 0 is
    taken), under the reference's checkpoint names and layouts.  Returns (config, weights,
    metadata).  ``w_x_offdiag`` fills W_x off its diagonal (the reference uses only the diagonal)."""
    d, H, V = mc.d, mc.H, mc.V
    ex: Dict[str, np.ndarray] = {}
    for n in ("w_q", "w_k", "w_v", "w_o", "w_in"):
        ex[f"reasoning.{n}"] = w[n][0].reshape(-1)
    wx = np.zeros((d, d), np.float32) if w_x_offdiag is None else np.array(w_x_offdiag, np.float32)
    np.fill_diagonal(wx, w["wx_diag"][0])
    ex["reasoning.w_x"] = wx.reshape(-1)
    ex["reasoning.w_out"] = (w["w_out"][0] if w.get("w_out") is not None else np.zeros((d, d), np.float32)).reshape(-1)
    for src, dst in (("q_bias", "q_bias"), ("k_bias", "k_bias")):
        ex[f"reasoning.{dst}"] = (w[src] if w.get(src) is not None else np.zeros((H, d), np.float32)).reshape(-1)
    ex["reasoning.slot_anchor"] = w["anchor"].reshape(-1)
    ex["reasoning.a_log"] = w["a_log"].reshape(-1)
    ex["reasoning.norm_scale"] = w["norm_scale"].reshape(-1)
    ex["reasoning.b_delta"] = (w["b_delta"][0] if w.get("b_delta") is not None else np.zeros(d, np.float32))
    if w.get("w_kw") is not None and w["w_kw"].shape[-1] == RETAIN_RANK:
        ex["reasoning.w_k_write"] = w["w_kw"].reshape(-1)
        ex["reasoning.w_v_write"] = w["w_vw"].reshape(-1)
    if w.get("w_hist") is not None:
        ex["reasoning.w_hist_shared"] = w["w_hist"].reshape(-1)
        ex["reasoning.hist_slot_scale"] = w["hist_slot_scale"].reshape(-1)
        ex["reasoning.hist_slot_bias"] = np.zeros(H * d, np.float32)
        ex["reasoning.hist_gate_logit"] = w["hist_gate_logit"].reshape(-1)
    ex["reasoning.damping"] = np.array([damping], np.float32)
    ex["reasoning.residual_alpha"] = np.array([0.0], np.float32)
    ex["head.w"] = w["lm_w"].reshape(-1)
    ex["head.b"] = (w["lm_b"] if w.get("lm_b") is not None else np.zeros(V, np.float32)).reshape(-1)
    ex["head.g"] = (w["lm_g"] if w.get("lm_g") is not None else np.ones(d, np.float32)).reshape(-1)
    # nalgebra stores the [V][d] table column-major: as_slice() is [d][V]
    ex["tokenizer.embeddings"] = np.ascontiguousarray(w["embed"].T).reshape(-1)
    config = dict(d_r=d, h_slots=H, vocab_size=V, ctx_len=512, max_deq_iters=mc.max_iters, deq_epsilon=mc.eps)
    metadata = {"aideen_version": "0.1.0", "type": "FullModel", "vocab_size": str(V)}
    return config, ex, metadata


class AidnConfig(C.Structure):
    _fields_ = [(n, C.c_float if c == "f" else (C.c_int32 if c == "?" else C.c_int64)) for n, c in CONFIG_FIELDS]


class AidnModel:
    """A checkpoint parsed by the library (host memory; no device is used)."""

    def __init__(self, path: str):
        from . import _lib
        self._L = _lib.lib()
        self._h = C.c_void_p()
        _lib.check(self._L.adn_aidn_open(path.encode(), C.byref(self._h)))

    def close(self) -> None:
        if self._h:
            self._L.adn_aidn_close(self._h)
            self._h = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def config(self) -> dict:
        from . import _lib
        c = AidnConfig()
        _lib.check(self._L.adn_aidn_config_get(self._h, C.byref(c)))
        return {n: getattr(c, n) for n, _ in CONFIG_FIELDS}

    def names(self):
        from . import _lib
        nw = C.c_int32()
        _lib.check(self._L.adn_aidn_count(self._h, C.byref(nw), None))
        out = []
        for i in range(nw.value):
            p = C.c_char_p()
            _lib.check(self._L.adn_aidn_name(self._h, i, C.byref(p)))
            out.append(p.value.decode())
        return out

    def tensor(self, name: str) -> Optional[np.ndarray]:
        from . import _lib
        p = C.POINTER(C.c_float)()
        n = C.c_int64()
        _lib.check(self._L.adn_aidn_tensor(self._h, name.encode(), C.byref(p), C.byref(n)))
        return np.ctypeslib.as_array(p, shape=(n.value,)).copy() if p else None

    def metadata(self, key: str) -> Optional[str]:
        from . import _lib
        p = C.c_char_p()
        _lib.check(self._L.adn_aidn_metadata(self._h, key.encode(), C.byref(p)))
        return None if p.value is None else p.value.decode()

    def weights(self):
        """(weights in this library's layout, adn_config fields, run defaults), copied out."""
        from . import _lib
        w = _lib.AdnWeights()
        cfg = _lib.AdnConfig()
        run = _lib.AdnRun()
        _lib.check(self._L.adn_aidn_weights(self._h, C.byref(w), C.byref(cfg), C.byref(run)))
        d, H, V, r = cfg.d_r, cfg.h_slots, cfg.vocab, cfg.rank
        shapes = dict(w_q=(H, d, d), w_k=(H, d, d), w_v=(H, d, d), w_o=(H, d, d), w_in=(H, d, d),
                      q_bias=(H, d), k_bias=(H, d), anchor=(H, d), norm_scale=(d,), embed=(V, d),
                      lm_w=(V, d), lm_b=(V,), lm_g=(d,), a_log=(H, d), wx_diag=(H, d), w_out=(H, d, d),
                      b_delta=(H, d), w_kw=(H, d, r), w_vw=(H, r, d), w_b=None, w_c=None,
                      w_hist=(d, d), hist_slot_scale=(H, d), hist_gate_logit=(H,))
        out = {}
        for name in _lib.WEIGHT_FIELDS:
            p = getattr(w, name)
            out[name] = None if not p or shapes[name] is None else \
                np.ctypeslib.as_array(p, shape=shapes[name]).copy()
        config = {f: getattr(cfg, f) for f, _ in cfg._fields_}
        run_defaults = dict(max_iters=run.max_iters, eps=run.eps, damping=run.damping)
        return out, config, run_defaults
