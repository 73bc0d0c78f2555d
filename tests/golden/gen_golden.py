"""Writes the committed golden fixtures of the C1 plumbing config.

The reference holds no golden vectors for this path (its tests restate the math inline), so
the fixtures are produced by the pinned CPU oracle on the build's deterministic synthetic
model (aideen_amd/synth.py, weights seed 0, tokens seed 1).  Inputs are reproduced from their
seeds; the file stores a digest of the weights so a generator drift is detected.

Run: python tests/golden/gen_golden.py [fixture names]
"""
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from aideen_amd import synth  # noqa: E402
from oracle import pyoracle  # noqa: E402


def c1_case(name="C1", weights="preset", **overrides):
    p = synth.PRESETS[name]
    import dataclasses
    mc = dataclasses.replace(p["model"], **overrides)
    w = synth.weights_of_kind(weights, mc, seed=0)
    toks = synth.make_tokens(p["tokens"], p["B"], p["T"], mc.V, seed=1)
    return mc, w, toks


# c1_token_sensitive: the C1 shape on synth.make_token_sensitive_weights, whose outputs depend
# strongly on the token (the reference's initialisation is anchor-dominated: one arg-max for all
# 64 tokens), so a fixture comparison can fail on a per-token error.
CASES = {
    "c1_forward": dict(),
    "c1_anderson_m5": dict(anderson_m=5, sigma=0.7),
    "c1_token_sensitive": dict(weights="token_sensitive"),
}


def main(names=None):
    """Writes the named fixtures (default: every case)."""
    pyoracle.build()
    for fname, ov in CASES.items():
        if names and fname not in names:
            continue
        mc, w, toks = c1_case(**ov)
        out = pyoracle.Oracle(mc, w).forward(toks)
        meta = dict(config=mc.as_dict(), B=int(toks.shape[0]), T=int(toks.shape[1]),
                    weights_sha256=synth.weights_digest(w), weights_seed=0, tokens_seed=1,
                    weights=ov.get("weights", "preset"))
        np.savez_compressed(os.path.join(HERE, fname + ".npz"), tokens=toks, **out)
        with open(os.path.join(HERE, fname + ".json"), "w") as f:
            json.dump(meta, f, indent=1, sort_keys=True)
        print(fname, {k: v.shape for k, v in out.items()}, "iters", np.bincount(out["iters"].ravel()))


if __name__ == "__main__":
    main(sys.argv[1:])
