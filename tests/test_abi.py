"""The C-ABI library loads and exports every symbol declared in include/*.h;
host-only entry points (geometry, MoE config) behave like the reference's.
CPU only: nothing here launches device work."""
import re
from pathlib import Path

import pytest

from conftest import ROOT, load_golden

import kq_hip


def declared_functions():
    names = set()
    for h in sorted((ROOT / "include").glob("*.h")):
        text = h.read_text()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"\b(kq_[a-z0-9_]+)\s*\(", text):
            names.add(m.group(1))
    return sorted(names)


def exported_symbols(path: Path):
    import subprocess
    out = subprocess.run(["nm", "-D", "--defined-only", str(path)], check=True,
                         capture_output=True, text=True).stdout
    return {line.split()[-1] for line in out.splitlines() if " T " in line}


def test_library_exports_every_declared_function():
    kq_hip.lib()  # loads (and binds every signature) or raises
    decl = declared_functions()
    assert len(decl) >= 25
    exported = exported_symbols(kq_hip.LIB_PATH)
    missing = [n for n in decl if n not in exported]
    assert missing == []
    # the binding declares exactly the header's functions
    assert sorted(kq_hip.SIGNATURES) == decl
    # internal launchers and helpers stay hidden
    assert not any(s.startswith(("kq_launch", "kqi_", "kq_fail")) for s in exported)


def test_geometry_matches_reference_table():
    # src/kq_gguf.c:57-65 (the reference's fixture table) plus Q6_K (256, 210).
    table = load_golden("numeric_vectors.json")["type_geometry"]
    for name, g in table.items():
        assert kq_hip.geometry(kq_hip.TYPE_IDS[name]) == (g["elements_per_block"],
                                                          g["bytes_per_block"]), name
    assert kq_hip.geometry(kq_hip.TYPE_Q6_K) == (256, 210)
    with pytest.raises(kq_hip.KqError) as e:
        kq_hip.geometry(2)  # Q4_0: no decode here
    assert e.value.name == "UNSUPPORTED_TENSOR_TYPE"


def test_packed_size_and_member_span():
    assert kq_hip.packed_size(kq_hip.TYPE_Q4_K, 4096 * 2048) == 4_718_592
    assert kq_hip.packed_size(kq_hip.TYPE_Q6_K, 151936 * 2048) == 255_252_480
    assert kq_hip.packed_size(kq_hip.TYPE_Q8_0, 4096 * 2048) == 8_912_896
    with pytest.raises(kq_hip.KqError) as e:
        kq_hip.packed_size(kq_hip.TYPE_Q4_K, 100)
    assert e.value.name == "INVALID_QUANTIZED_GEOMETRY"
    # expert e's gate in a [512][512][2048] Q4_K stack: e * 589,824 bytes
    assert kq_hip.expert_member_span(kq_hip.TYPE_Q4_K, 512, 2048, 512, 7) == (7 * 589_824, 589_824)
    assert kq_hip.expert_member_span(kq_hip.TYPE_Q6_K, 2048, 512, 512, 511) == (511 * 860_160,
                                                                             860_160)
    with pytest.raises(kq_hip.KqError) as e:
        kq_hip.expert_member_span(kq_hip.TYPE_Q4_K, 512, 2048, 512, 512)
    assert e.value.name == "SPAN_OUT_OF_RANGE"


def test_moe_config_validation_and_scratch():
    cfg = kq_hip.MoeConfig(2048, 512, 10, 512, 512)
    s1 = cfg.scratch_bytes(1)
    s512 = cfg.scratch_bytes(512)
    assert 0 < s1 < s512
    with pytest.raises(kq_hip.KqError) as e:
        kq_hip.MoeConfig(2048, 4, 5, 512, 512)  # top_k > experts
    assert e.value.name == "INCOMPATIBLE_MOE"
    with pytest.raises(kq_hip.KqError) as e:
        kq_hip.MoeConfig(0, 4, 2, 4, 4)
    assert e.value.name == "INCOMPATIBLE_MOE"
    with pytest.raises(kq_hip.KqError) as e:
        kq_hip.MoeConfig(2048, 2048, 10, 512, 512)  # beyond the device router's 1023 experts
    assert e.value.name == "LIMIT_EXCEEDED"


def test_status_strings():
    lib = kq_hip.lib()
    assert lib.kq_status_string(0) == b"ok"
    assert lib.kq_status_string(38) == b"malformed quantized data"
    assert lib.kq_status_string(1000) == b"device failure"
    # every code the binding names has its own string
    strings = {lib.kq_status_string(code) for code in kq_hip.STATUS}
    assert len(strings) == len(kq_hip.STATUS) and b"unknown status" not in strings
    assert lib.kq_status_string(29) == b"unknown status"  # a tokenizer code, not on this path


def _gpu_present() -> bool:
    import os
    return os.path.exists("/dev/kfd") and any(Path("/dev/dri").glob("renderD*"))


@pytest.mark.skipif(_gpu_present(), reason="checks the no-device path")
def test_context_fails_loudly_without_a_device():
    with pytest.raises(kq_hip.KqError) as e:
        kq_hip.Context(0)
    assert e.value.name == "DEVICE_FAILURE"
