"""`.aidn` checkpoints: the bincode 1.3 format (aideen-core/src/model.rs:10-58, state.rs:7-35) and
the mapping of the reference's names and layouts onto the library's weights.  CPU only: the
library's loader touches no device.

bincode 1.3.3 is a dependency the reference pins (Cargo.lock) but that is absent here, so the
format is pinned by a byte string assembled by hand from its published encoding rules (u64
little-endian lengths and integers, bool as one byte, struct fields in declaration order, maps
as a count and key/value pairs), by the Python encoder/decoder, and by round trips through the
C++ loader.
"""
import dataclasses
import os

import numpy as np
import pytest

from aideen_amd import aidn, synth
from aideen_amd._lib import AdnError

# A tiny AidenModel by hand: config d_m=1, d_r=2, d_c=3, d_e=4, d_sim=5, h_slots=6, vocab=7,
# ctx_len=8, max_deq_iters=9, deq_epsilon=0.5, adj_iters=10, train_deq=true, deq_grad_scale=2.0,
# renorm_every_steps=11, num_samples=12, weight_decay=0.25; weights {"w": [1.5, -2.0]};
# metadata {"k": "vé"} (UTF-8, 3 bytes).
KNOWN = bytes.fromhex(
    "0100000000000000" "0200000000000000" "0300000000000000" "0400000000000000" "0500000000000000"
    "0600000000000000" "0700000000000000" "0800000000000000" "0900000000000000"
    "0000003f"                      # 0.5f
    "0a00000000000000" "01"         # adj_iters, train_deq
    "00000040"                      # 2.0f
    "0b00000000000000" "0c00000000000000"
    "0000803e"                      # 0.25f
    "0100000000000000" "0100000000000000" "77" "0200000000000000" "0000c03f" "000000c0"
    "0100000000000000" "0100000000000000" "6b" "0300000000000000" "76c3a9")


def test_known_bytes_python_decoder():
    cfg, w, meta = aidn.decode(KNOWN)
    assert cfg["d_m"] == 1 and cfg["d_r"] == 2 and cfg["max_deq_iters"] == 9 and cfg["num_samples"] == 12
    assert cfg["deq_epsilon"] == 0.5 and cfg["train_deq"] is True and cfg["weight_decay"] == 0.25
    assert list(w) == ["w"] and np.array_equal(w["w"], np.array([1.5, -2.0], np.float32))
    assert meta == {"k": "vé"}
    assert aidn.encode(cfg, w, meta) == KNOWN


def test_known_bytes_library_loader(tmp_path):
    p = str(tmp_path / "k.aidn")
    open(p, "wb").write(KNOWN)
    m = aidn.AidnModel(p)
    c = m.config()
    assert (c["d_m"], c["d_r"], c["d_c"], c["d_e"], c["d_sim"], c["h_slots"], c["vocab_size"], c["ctx_len"],
            c["max_deq_iters"], c["adj_iters"], c["renorm_every_steps"], c["num_samples"]) == \
        (1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12)
    assert (c["deq_epsilon"], c["train_deq"], c["deq_grad_scale"], c["weight_decay"]) == (0.5, 1, 2.0, 0.25)
    assert m.names() == ["w"]
    assert np.array_equal(m.tensor("w"), np.array([1.5, -2.0], np.float32))
    assert m.tensor("absent") is None
    assert m.metadata("k") == "vé" and m.metadata("x") is None


@pytest.mark.parametrize("cut", [1, 3, 20, 60])
def test_corrupt_files_are_rejected(tmp_path, cut):
    p = str(tmp_path / "t.aidn")
    open(p, "wb").write(KNOWN[:-cut])
    with pytest.raises(AdnError, match="truncated"):
        aidn.AidnModel(p)
    open(p, "wb").write(KNOWN + b"\0")
    with pytest.raises(AdnError, match="trailing"):
        aidn.AidnModel(p)
    with pytest.raises(AdnError, match="cannot open"):
        aidn.AidnModel(str(tmp_path / "missing.aidn"))
    # a length far beyond the file must not allocate, only fail
    bad = bytearray(KNOWN)
    bad[109:117] = (1 << 40).to_bytes(8, "little")  # the weight count
    open(p, "wb").write(bytes(bad))
    with pytest.raises(AdnError):
        aidn.AidnModel(p)


def shared_model(mc, seed=3, hist=True):
    """synth weights with every slot sharing the matrices the CPU model shares."""
    w = dict(synth.make_weights(mc, seed=seed))
    for n in ("w_q", "w_k", "w_v", "w_o", "w_in", "w_out", "wx_diag", "b_delta"):
        w[n] = np.ascontiguousarray(np.repeat(w[n][:1], mc.H, axis=0))
    if hist:
        w.update(synth.make_hist_weights(mc, seed=seed, strong=True))
    return w


def test_reference_layout_round_trip(tmp_path):
    mc = synth.ModelConfig(d=64, H=4, V=300, N=1, r=32, flags=0, qk_bias=True)
    w = shared_model(mc)
    rng = np.random.default_rng(0)
    offdiag = rng.standard_normal((mc.d, mc.d)).astype(np.float32)
    cfg, ex, meta = aidn.reference_export(mc, w, damping=0.65, w_x_offdiag=offdiag)
    p = str(tmp_path / "m.aidn")
    aidn.write_aidn(p, cfg, ex, meta)
    # the Python reader and the library agree on every tensor
    c2, ex2, meta2 = aidn.read_aidn(p)
    m = aidn.AidnModel(p)
    assert sorted(m.names()) == sorted(ex) and m.metadata("vocab_size") == "300"
    for k, v in ex.items():
        assert np.array_equal(m.tensor(k), v) and np.array_equal(ex2[k], v), k
    got, acfg, run = m.weights()
    assert (acfg["d_r"], acfg["h_slots"], acfg["vocab"], acfg["d_state"], acfg["rank"]) == (64, 4, 300, 1, 32)
    assert acfg["flags"] == 0 and acfg["max_seq"] == cfg["ctx_len"]
    assert run["max_iters"] == mc.max_iters and np.float32(run["eps"]) == np.float32(mc.eps)
    assert np.float32(run["damping"]) == np.float32(0.65)
    for n in ("w_q", "w_k", "w_v", "w_o", "w_in", "w_out", "wx_diag", "b_delta", "q_bias", "k_bias",
              "anchor", "norm_scale", "embed", "lm_w", "lm_b", "lm_g", "a_log", "w_kw", "w_vw", "w_hist",
              "hist_slot_scale", "hist_gate_logit"):
        assert np.array_equal(got[n], w[n]), n
    assert got["w_b"] is None and got["w_c"] is None


def test_missing_and_mismatched_tensors(tmp_path):
    mc = synth.ModelConfig(d=64, H=2, V=100, N=1, r=32, flags=0)
    w = shared_model(mc, hist=False)
    cfg, ex, meta = aidn.reference_export(mc, w)
    p = str(tmp_path / "m.aidn")
    for drop, msg in (("reasoning.w_q", "reasoning.w_q not found"), ("head.w", "head.w not found"),
                      ("reasoning.slot_anchor", "slot_anchor"), ("tokenizer.embeddings", "embeddings")):
        e2 = dict(ex)
        del e2[drop]
        aidn.write_aidn(p, cfg, e2, meta)
        with pytest.raises(AdnError, match=msg):
            aidn.AidnModel(p).weights()
    e2 = dict(ex)
    e2["reasoning.w_o"] = e2["reasoning.w_o"][:-1]
    aidn.write_aidn(p, cfg, e2, meta)
    with pytest.raises(AdnError, match="w_o size mismatch"):
        aidn.AidnModel(p).weights()
    # optional tensors may be absent: no biases, no history weights
    e2 = {k: v for k, v in ex.items() if k not in ("reasoning.q_bias", "reasoning.k_bias")}
    aidn.write_aidn(p, cfg, e2, meta)
    got, _, _ = aidn.AidnModel(p).weights()
    assert got["q_bias"] is None and got["w_hist"] is None


def test_metadata_vocab_size_wins(tmp_path):
    """The trainer sizes the vocabulary from metadata["vocab_size"] (trainer.rs:6607-6616)."""
    mc = synth.ModelConfig(d=64, H=2, V=120, N=1, r=32, flags=0)
    w = shared_model(mc, hist=False)
    cfg, ex, meta = aidn.reference_export(mc, w)
    cfg["vocab_size"] = 50257
    p = str(tmp_path / "m.aidn")
    aidn.write_aidn(p, cfg, ex, meta)
    got, acfg, _ = aidn.AidnModel(p).weights()
    assert acfg["vocab"] == 120 and got["embed"].shape == (120, 64)


@pytest.mark.parametrize("config,meta,match", [
    (dict(d_r=64, h_slots=(1 << 58) + 1), {}, "h_slots"),      # H*d would wrap to 64 without bounds
    (dict(d_r=4096, h_slots=1), {}, "d_r"),
    (dict(d_r=64, h_slots=2, vocab_size=1 << 40), {}, "vocab_size"),
    (dict(d_r=64, h_slots=2, vocab_size=10), {"vocab_size": "12x"}, "vocab_size"),
    (dict(d_r=64, h_slots=2, vocab_size=10), {"vocab_size": "99999999999999999999"}, "vocab_size"),
])
def test_crafted_header_sizes_are_rejected(tmp_path, config, meta, match):
    """Sizes from an untrusted header are bounded before any product of them is formed, so a tiny
    file cannot pass the size checks through a wrapped product (an overflow of the per-slot
    copies), and a malformed metadata vocabulary is refused."""
    p = str(tmp_path / "crafted.aidn")
    d = 64
    w = {"reasoning.w_q": np.zeros(d * d, np.float32), "reasoning.slot_anchor": np.zeros(2 * d, np.float32)}
    aidn.write_aidn(p, config, w, meta)
    m = aidn.AidnModel(p)
    with pytest.raises(AdnError, match=match):
        m.weights()
    m.close()
