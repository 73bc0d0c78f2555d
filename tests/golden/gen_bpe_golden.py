"""Golden vectors for the byte-level BPE encoder/decoder.

The reference encodes with the HF `tokenizers` crate (0.21.4 in its Cargo.lock) loading
aideen-backbone/tokenizer.json (tokenizer.rs:53-104: encode(text, add_special_tokens = true),
decode(ids, skip_special_tokens = true)).  This script runs the same library (its Python
binding, as installed in the build container) on the same file and records ids and decoded
text for a fixed set of inputs plus seeded random strings over many scripts.  Run from the
repository root: python tests/golden/gen_bpe_golden.py [path/to/tokenizer.json]
"""
import hashlib
import json
import os
import random
import sys

import tokenizers

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = sys.argv[1] if len(sys.argv) > 1 else "/root/reference/aideen-backbone/tokenizer.json"

FIXED = [
    "", "a", " ", "  ", "\n", "hello world", "Hello, World!", "hola mundo",
    "It's a test. They're here, we've seen, I'm sure, you'll see, he'd go.",
    "'s 't 're 've 'm 'll 'd", "'S 'T 'RE", "don't won't can't",
    "1234567890", "3.14159 + 2.71828 = 5.85987", "x1y2z3 v2.0 AB-12",
    "a  b   c    d", "trailing   ", "   leading", "tabs\tand\nnewlines\r\nand\u000bvertical",
    "a\n b", "a \nb", "a\n\n\nb", "end with newline\n", " \n \n ",
    "café naïve résumé Ångström", "Привет мир", "こんにちは世界", "你好，世界！", "안녕하세요",
    "مرحبا بالعالم", "שלום עולם", "नमस्ते दुनिया", "Ελληνικά", "🙂😀 emoji 👍🏽 family 👨‍👩‍👧",
    "mixed: abcÄÖÜ123٤٥٦ and Ⅻ ½ ²", "non breaking em　ideographic",
    "<|endoftext|>", "before<|endoftext|>after", "a <|endoftext|> b<|endoftext|><|endoftext|>",
    "<|endoftext", "punctuation!!! ??? ... ,,, ;;; --- ___ @@@ ### $$$ %%% ^^^ &&& ***",
    "math: ∑∫√∞≠≤≥ ∂x/∂y", "code: def f(x):\n    return x**2  # square\n",
    "url https://example.com/path?q=1&r=2#frag and email a.b@c.de",
    "ZWJ‍and‌ZWNJ and soft­hyphen", "control \u0001\u0002\u007f chars",
    "The quick brown fox jumps over the lazy dog. " * 20,
]

POOLS = [
    (0x20, 0x7E), (0xA0, 0x24F), (0x370, 0x3FF), (0x400, 0x4FF), (0x590, 0x6FF), (0x900, 0x97F),
    (0x3040, 0x30FF), (0x4E00, 0x4FFF), (0xAC00, 0xAD00), (0x2000, 0x206F), (0x2150, 0x218F),
    (0x1F300, 0x1F64F), (0x9, 0xD),
]


def random_texts(n, seed=7):
    rng = random.Random(seed)
    out = []
    for _ in range(n):
        k = rng.randint(1, 60)
        s = []
        for _ in range(k):
            lo, hi = rng.choice(POOLS)
            s.append(chr(rng.randint(lo, hi)) if rng.random() < 0.7 else rng.choice([" ", " ", "  ", "'s", "'ll", "\n"]))
        out.append("".join(s))
    return out


def main():
    tok = tokenizers.Tokenizer.from_file(SRC)
    texts = FIXED + random_texts(300)
    cases = []
    for t in texts:
        enc = tok.encode(t, add_special_tokens=True)
        cases.append(dict(text=t, ids=enc.ids, decoded=tok.decode(enc.ids, skip_special_tokens=True)))
    # decode of id runs cut inside multi-byte characters (lossy UTF-8) and with special ids
    rng = random.Random(11)
    decode_cases = []
    for c in cases:
        ids = c["ids"]
        if len(ids) < 3:
            continue
        a = rng.randrange(0, len(ids) - 1)
        b = rng.randrange(a + 1, len(ids) + 1)
        cut = ids[a:b] + ([50256] if rng.random() < 0.3 else [])
        decode_cases.append(dict(ids=cut, decoded=tok.decode(cut, skip_special_tokens=True)))
    meta = dict(tokenizers_python=tokenizers.__version__,
                tokenizer_json_sha256=hashlib.sha256(open(SRC, "rb").read()).hexdigest(),
                vocab_size=tok.get_vocab_size(True))
    json.dump(dict(meta=meta, cases=cases, decode_cases=decode_cases), open(os.path.join(HERE, "bpe_golden.json"), "w"),
              ensure_ascii=False, indent=0)
    print(f"{len(cases)} cases, {sum(len(c['ids']) for c in cases)} ids")


if __name__ == "__main__":
    main()
