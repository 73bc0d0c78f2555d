"""The library's byte-level BPE tokenizer (``adn_tokenizer_*``) under the reference's method names
(Tokenizer::encode / decode / vocab_size, tokenizer.rs:85-116)."""
from __future__ import annotations

import ctypes as C
from typing import List, Sequence

import numpy as np

from . import _lib


class BpeTokenizer:
    def __init__(self, tokenizer_json: str):
        self._L = _lib.lib()
        self._h = C.c_void_p()
        _lib.check(self._L.adn_tokenizer_load(tokenizer_json.encode(), C.byref(self._h)))

    def close(self) -> None:
        if self._h:
            self._L.adn_tokenizer_free(self._h)
            self._h = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def vocab_size(self) -> int:
        return int(self._L.adn_tokenizer_vocab_size(self._h))

    def encode(self, text: str) -> List[int]:
        b = text.encode("utf-8")
        n = C.c_int64()
        cap = len(b) + 8  # byte-level BPE: at most one id per byte, plus added tokens
        ids = np.zeros(cap, np.int32)
        _lib.check(self._L.adn_tokenizer_encode(self._h, b, len(b), ids.ctypes.data_as(_lib.I32P), cap,
                                                C.byref(n)))
        return ids[:n.value].tolist()

    def decode(self, ids: Sequence[int]) -> str:
        a = np.ascontiguousarray(np.asarray(ids, dtype=np.int32))
        n = C.c_int64()
        cap = 4 * len(a) * 8 + 16
        buf = C.create_string_buffer(cap)
        _lib.check(self._L.adn_tokenizer_decode(self._h, a.ctypes.data_as(_lib.I32P), len(a), buf, cap,
                                                C.byref(n)))
        return buf.raw[:n.value].decode("utf-8")
