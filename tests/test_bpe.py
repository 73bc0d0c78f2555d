"""Byte-level BPE encode/decode (the library's adn_tokenizer_*) against golden vectors of the HF
`tokenizers` library on the reference's tokenizer.json (tests/golden/gen_bpe_golden.py).  CPU
only.  The tokenizer file is the reference's data (aideen-backbone/tokenizer.json): its path is
taken from AIDEEN_TOKENIZER_JSON or the reference checkout, and the tests skip without it.
Bar: identical ids and identical decoded text."""
import hashlib
import json
import os

import numpy as np
import pytest

from aideen_amd._lib import AdnError

HERE = os.path.dirname(os.path.abspath(__file__))
GOLDEN = json.load(open(os.path.join(HERE, "golden", "bpe_golden.json"), encoding="utf-8"))
PATH = os.environ.get("AIDEEN_TOKENIZER_JSON", "/root/reference/aideen-backbone/tokenizer.json")

pytestmark = pytest.mark.skipif(not os.path.exists(PATH), reason="tokenizer.json not available")


@pytest.fixture(scope="module")
def tok():
    assert hashlib.sha256(open(PATH, "rb").read()).hexdigest() == GOLDEN["meta"]["tokenizer_json_sha256"]
    from aideen_amd.tokenizer import BpeTokenizer
    return BpeTokenizer(PATH)


def test_vocab_size(tok):
    assert tok.vocab_size() == GOLDEN["meta"]["vocab_size"] == 50257


def test_encode_matches_golden(tok):
    bad = [(c["text"], tok.encode(c["text"]), c["ids"]) for c in GOLDEN["cases"] if tok.encode(c["text"]) != c["ids"]]
    assert not bad, f"{len(bad)} mismatches, first: {bad[0]!r}"


def test_decode_matches_golden(tok):
    for c in GOLDEN["cases"]:
        assert tok.decode(c["ids"]) == c["decoded"], c["text"]
    for c in GOLDEN["decode_cases"]:
        assert tok.decode(c["ids"]) == c["decoded"], c["ids"]


def test_round_trip_and_special(tok):
    s = "Round trip: ünïcödé, 数字 123, emoji 🙂 and <|endoftext|> inside."
    ids = tok.encode(s)
    assert 50256 in ids
    assert tok.decode(ids) == s.replace("<|endoftext|>", "")  # special tokens are skipped
    assert tok.decode([]) == "" and tok.encode("") == []
    assert tok.decode([99999999, -1, 64]) == "a"  # ids without a token are skipped


def test_errors(tok, tmp_path):
    from aideen_amd import _lib
    import ctypes as C
    L = _lib.lib()
    n = C.c_int64()
    ids = np.zeros(2, np.int32)
    rc = L.adn_tokenizer_encode(tok._h, b"\xff\xfe", 2, ids.ctypes.data_as(_lib.I32P), 2, C.byref(n))
    assert rc == _lib.ADN_E_INVALID and b"UTF-8" in L.adn_last_error()
    rc = L.adn_tokenizer_encode(tok._h, b"hello world again", 17, ids.ctypes.data_as(_lib.I32P), 2, C.byref(n))
    assert rc == _lib.ADN_E_CAPACITY and n.value == 3
    j = json.load(open(PATH, encoding="utf-8"))
    j["pre_tokenizer"]["add_prefix_space"] = True
    p = tmp_path / "t.json"
    p.write_text(json.dumps(j), encoding="utf-8")
    from aideen_amd.tokenizer import BpeTokenizer
    with pytest.raises(AdnError, match="prefix space"):
        BpeTokenizer(str(p))
    p.write_text("{\"model\": [1, 2", encoding="utf-8")
    with pytest.raises(AdnError, match="tokenizer.json"):
        BpeTokenizer(str(p))
