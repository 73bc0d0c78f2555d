"""C-ABI library checks that need no GPU: it loads, exports every declared symbol, and its
host-side validation rejects bad configurations before touching a device."""
import ctypes as C
import re

import pytest

from aideen_amd import _lib, synth


def test_library_loads_and_exports_every_header_symbol():
    L = _lib.lib()
    names = _lib.header_functions()
    assert len(names) >= 15
    for n in names:
        assert hasattr(L, n), f"{n} declared in include/aideen_hip.h but not exported"
    assert L.adn_abi_version() == 3


def test_header_flag_values_match_oracle_and_synth():
    text = open(_lib.HEADER).read()
    hdr = {m.group(1): int(m.group(2)) for m in re.finditer(r"#define ADN_F_(\w+) \(1u << (\d+)\)", text)}
    orc = open(_lib.HEADER.replace("include/aideen_hip.h", "oracle/aideen_oracle.h")).read()
    ohd = {m.group(1): int(m.group(2)) for m in re.finditer(r"#define ORC_F_(\w+)\s+\(1u << (\d+)\)", orc)}
    # semantic switches are shared with the oracle; the GEMM arithmetic bits are product-only
    assert {k: v for k, v in hdr.items() if not k.startswith("GEMM_")} == ohd
    for k, v in hdr.items():
        assert getattr(synth, "F_" + k) == 1 << v


def test_struct_layouts_match_header():
    # field order and count of the ctypes mirrors == the C structs
    text = open(_lib.HEADER).read()
    body = re.search(r"typedef struct adn_weights \{(.*?)\} adn_weights;", text, re.S).group(1)
    fields = re.findall(r"\*(\w+)", body)
    assert fields == _lib.WEIGHT_FIELDS
    assert C.sizeof(_lib.AdnConfig) == 9 * 4
    assert C.sizeof(_lib.AdnWeights) == 24 * 8


@pytest.mark.parametrize("bad", [
    dict(d_r=100), dict(d_r=4096), dict(d_r=0), dict(h_slots=0), dict(h_slots=17), dict(d_state=0), dict(d_state=64),
    dict(rank=0), dict(max_batch=0), dict(anderson_m=6), dict(flags=1 << 13), dict(flags=(1 << 4) | (1 << 11)),
    dict(flags=1 << 10, d_state=1),
    dict(flags=1 << 9, d_state=4),
    dict(flags=(1 << 9) | (1 << 5), d_state=1), dict(vocab=0), dict(flags=(1 << 6) | (1 << 7)),
])
def test_create_rejects_invalid_config_before_device(bad):
    L = _lib.lib()
    base = dict(d_r=128, h_slots=4, vocab=512, d_state=16, rank=32, max_batch=1, max_seq=8,
                anderson_m=0, flags=0)
    base.update(bad)
    cfg = _lib.AdnConfig(**base)
    ctx = C.c_void_p()
    rc = L.adn_create(C.byref(cfg), C.byref(ctx))
    assert rc == _lib.ADN_E_INVALID
    assert L.adn_last_error().decode()
    assert not ctx.value


def test_null_arguments_are_errors():
    L = _lib.lib()
    assert L.adn_create(None, None) == _lib.ADN_E_INVALID
    assert L.adn_synchronize(None) == _lib.ADN_E_INVALID
    assert L.adn_forward(None, None, None) == _lib.ADN_E_INVALID
    assert L.adn_lm_sample(None, 1, 10, None, None, 0, None, 0.8, 0.9, 40, 1.1, None, None) == _lib.ADN_E_INVALID
    assert L.adn_decode_sample(None, 1, 1, None, 1, 1, 10, 0.0, 0.7, 0.8, 0.9, 40, 1.1, None,
                               None) == _lib.ADN_E_INVALID
    L.adn_destroy(None)


def test_integration_ffi_block_binds_every_header_symbol():
    """The integration guide's `extern "C"` block (the Rust -sys crate a maintainer adds) declares every
    function the header does, and nothing else."""
    import os
    text = open(os.path.join(os.path.dirname(_lib.HEADER), "..", "INTEGRATION.md")).read()
    block = text[text.index('extern "C" {'):]
    block = block[:block.index("\n}\n")]
    names = sorted(set(re.findall(r"pub fn (adn_\w+)\s*\(", block)))
    assert names == _lib.header_functions()
