"""ctypes binding of libaideen_hip.so (the C ABI in include/aideen_hip.h).

Loading fails loudly when the library has not been built: there is no CPU fallback.
"""
from __future__ import annotations

import ctypes as C
import os
import re

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libaideen_hip.so")
HEADER = os.path.join(os.path.dirname(HERE), "include", "aideen_hip.h")

ADN_OK = 0
ADN_E_INVALID = -1
ADN_E_NO_DEVICE = -2
ADN_E_HIP = -3
ADN_E_NO_WEIGHTS = -4
ADN_E_CAPACITY = -5

ADN_LAYOUT_OUT_IN = 0
ADN_LAYOUT_IN_OUT = 1

F32P = C.POINTER(C.c_float)
I32P = C.POINTER(C.c_int32)


class AdnConfig(C.Structure):
    _fields_ = [("d_r", C.c_int32), ("h_slots", C.c_int32), ("vocab", C.c_int32),
                ("d_state", C.c_int32), ("rank", C.c_int32), ("max_batch", C.c_int32),
                ("max_seq", C.c_int32), ("anderson_m", C.c_int32), ("flags", C.c_uint32)]


WEIGHT_FIELDS = ["w_q", "w_k", "w_v", "w_o", "w_in", "q_bias", "k_bias", "anchor", "norm_scale",
                 "embed", "lm_w", "lm_b", "lm_g", "a_log", "wx_diag", "w_out", "b_delta", "w_kw",
                 "w_vw", "w_b", "w_c", "w_hist", "hist_slot_scale", "hist_gate_logit"]


class AdnWeights(C.Structure):
    _fields_ = [(n, F32P) for n in WEIGHT_FIELDS]


class AdnRun(C.Structure):
    _fields_ = [("batch", C.c_int32), ("seq", C.c_int32), ("max_iters", C.c_int32),
                ("eps", C.c_float), ("damping", C.c_float), ("tokens", I32P), ("s_in", F32P),
                ("scan_state_in", F32P)]


class AdnOutputs(C.Structure):
    _fields_ = [("h_star", F32P), ("pooled", F32P), ("logits", F32P), ("argmax", I32P),
                ("iters", I32P), ("scan_y", F32P), ("scan_state", F32P), ("converged", I32P)]


STAGES = ["signal_gemm", "init", "qkv_gemm", "attn", "wo_gemm", "update", "converge", "anderson",
          "pool", "lmhead_gemm", "argmax", "scan_prep", "scan", "readout_gemm", "hist_gemm", "hist_ctx",
          "temporal"]
PROFILE_MAX_ITERS = 256


class AdnProfile(C.Structure):
    _fields_ = [("ms", C.c_double * len(STAGES)), ("flops", C.c_double * len(STAGES)),
                ("bytes", C.c_double * len(STAGES)), ("launches", C.c_int32 * len(STAGES)),
                ("active", C.c_int32 * PROFILE_MAX_ITERS), ("n_iters", C.c_int32),
                ("total_ms", C.c_double)]


class AdnError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"[{code}] {msg}")
        self.code = code


_lib = None


def header_functions() -> list:
    """Names of every function the public header declares."""
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(adn_\w+)\s*\(", text, re.M)))


def lib():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"{LIB_PATH} is missing: build it with `python -m aideen_amd.build` "
            "(the HIP path has no CPU fallback)")
    L = C.CDLL(LIB_PATH)
    ctx_p = C.c_void_p
    sig = {
        "adn_abi_version": (C.c_int, []),
        "adn_last_error": (C.c_char_p, []),
        "adn_device_count": (C.c_int, [I32P]),
        "adn_create": (C.c_int, [C.POINTER(AdnConfig), C.POINTER(ctx_p)]),
        "adn_destroy": (None, [ctx_p]),
        "adn_set_stream": (C.c_int, [ctx_p, C.c_void_p]),
        "adn_synchronize": (C.c_int, [ctx_p]),
        "adn_upload_weights": (C.c_int, [ctx_p, C.POINTER(AdnWeights), C.c_uint32]),
        "adn_reset_state": (C.c_int, [ctx_p]),
        "adn_forward": (C.c_int, [ctx_p, C.POINTER(AdnRun), C.POINTER(AdnOutputs)]),
        "adn_forward_async": (C.c_int, [ctx_p, C.POINTER(AdnRun), C.POINTER(AdnOutputs)]),
        "adn_decode_greedy": (C.c_int, [ctx_p, C.c_int32, C.c_int32, I32P, C.c_int32, C.c_int32, C.c_int32,
                                        C.c_float, C.c_float, C.c_float, I32P]),
        "adn_lm_sample": (C.c_int, [ctx_p, C.c_int32, C.c_int32, F32P, I32P, C.c_int32, I32P, C.c_float, C.c_float,
                                    C.c_int32, C.c_float, F32P, I32P]),
        "adn_decode_sample": (C.c_int, [ctx_p, C.c_int32, C.c_int32, I32P, C.c_int32, C.c_int32, C.c_int32,
                                        C.c_float, C.c_float, C.c_float, C.c_float, C.c_int32, C.c_float, F32P,
                                        I32P]),
        "adn_spectral_norm": (C.c_int, [ctx_p, F32P, C.c_int32, C.c_int32, C.c_int32, F32P]),
        "adn_normalize_if_needed": (C.c_int, [ctx_p, F32P, C.c_int32, C.c_int32, C.c_float, C.c_int32]),
        "adn_renormalize_spectral": (C.c_int, [ctx_p, C.c_float, C.c_float, C.c_float, C.c_float, C.c_float,
                                               C.c_int32, F32P]),
        "adn_block_step": (C.c_int, [ctx_p, C.c_int32, F32P, F32P, F32P, F32P, F32P, F32P]),
        "adn_load_tensor": (C.c_int, [ctx_p, F32P, C.c_int64, I32P]),
        "adn_ffn_forward": (C.c_int, [ctx_p, C.c_int32, C.c_int32, C.c_int32, F32P]),
        "adn_adjoint": (C.c_int, [ctx_p, C.c_int32, F32P, F32P, C.c_int32, C.c_float, F32P, F32P]),
        "adn_adjoint_async": (C.c_int, [ctx_p, C.c_int32, F32P, F32P, C.c_int32, C.c_float, F32P, F32P]),
        "adn_tokenizer_load": (C.c_int, [C.c_char_p, C.POINTER(C.c_void_p)]),
        "adn_tokenizer_free": (None, [C.c_void_p]),
        "adn_tokenizer_vocab_size": (C.c_int32, [C.c_void_p]),
        "adn_tokenizer_encode": (C.c_int, [C.c_void_p, C.c_char_p, C.c_int64, I32P, C.c_int64,
                                           C.POINTER(C.c_int64)]),
        "adn_tokenizer_decode": (C.c_int, [C.c_void_p, I32P, C.c_int64, C.c_char_p, C.c_int64,
                                           C.POINTER(C.c_int64)]),
        "adn_aidn_open": (C.c_int, [C.c_char_p, C.POINTER(C.c_void_p)]),
        "adn_aidn_close": (None, [C.c_void_p]),
        "adn_aidn_config_get": (C.c_int, [C.c_void_p, C.c_void_p]),
        "adn_aidn_count": (C.c_int, [C.c_void_p, I32P, I32P]),
        "adn_aidn_name": (C.c_int, [C.c_void_p, C.c_int32, C.POINTER(C.c_char_p)]),
        "adn_aidn_tensor": (C.c_int, [C.c_void_p, C.c_char_p, C.POINTER(F32P), C.POINTER(C.c_int64)]),
        "adn_aidn_metadata": (C.c_int, [C.c_void_p, C.c_char_p, C.POINTER(C.c_char_p)]),
        "adn_aidn_weights": (C.c_int, [C.c_void_p, C.POINTER(AdnWeights), C.POINTER(AdnConfig),
                                       C.POINTER(AdnRun)]),
        "adn_embed_context": (C.c_int, [ctx_p, C.c_int32, C.c_int32, I32P, C.c_int32, F32P]),
        "adn_embed_context_async": (C.c_int, [ctx_p, C.c_int32, C.c_int32, I32P, C.c_int32, F32P]),
        "adn_embed_context_noalloc": (C.c_int, [ctx_p, C.c_int32, C.c_int32, I32P, C.c_int32, F32P]),
        "adn_noalloc_guard_set": (C.c_int, [ctx_p, C.c_uint32]),
        "adn_profile_forward": (C.c_int, [ctx_p, C.POINTER(AdnRun), C.POINTER(AdnOutputs),
                                          C.POINTER(AdnProfile)]),
    }
    for name, (res, args) in sig.items():
        f = getattr(L, name)
        f.restype = res
        f.argtypes = args
    _lib = L
    return L


def check(rc: int) -> None:
    if rc != ADN_OK:
        raise AdnError(rc, lib().adn_last_error().decode(errors="replace"))
