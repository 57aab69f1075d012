"""The sampler's host functions in libkq_hip.so, through the C ABI, no GPU:
the PCG32 RNG record (seed, next, reset, snapshot/import, integrity and
draw-count checks) against the reference's RNG vectors
(research/sampling, EXACT_BITS) and the oracle's generator, the default
policy, and the policy checks of config open, which come before any device
work (src/kq_sampling.c:161-225, :246-322)."""
import ctypes as C

import numpy as np
import pytest

from conftest import load_golden

import kq_hip
import kq_oracle

SV = load_golden("sampling_vectors.json")


def status_of(fn, *args):
    d = kq_hip.Diagnostic()
    return kq_hip.STATUS.get(fn(*args, C.byref(d)), "?"), d


def integrity(s) -> int:
    # FNV-1a-style mix of the record's seven fields (src/kq_sampling.c:83-96)
    h = 1469598103934665603
    for f in (s.version, s.reserved, s.seed, s.stream, s.state, s.increment, s.draws):
        h = ((h ^ f) * 1099511628211) % 2 ** 64
    return h


def test_rng_vectors_bit_exact():
    for c in SV["rng"]["cases"]:
        st = kq_hip.rng_seed(c["seed"], c["stream"])
        assert st.increment == int(c["increment_hex"], 16)
        assert st.state == int(c["seeded_state_hex"], 16)
        assert st.integrity == integrity(st)
        for w in c["words"]:
            assert kq_hip.rng_next(st) == int(w["word_hex"], 16)
            assert st.draws == w["draw"] and st.state == int(w["state_after_hex"], 16)
            assert st.integrity == integrity(st)


def test_rng_matches_oracle_stream():
    rng = np.random.default_rng(5)
    for _ in range(20):
        seed = int(rng.integers(0, 2 ** 63)) * 2 + int(rng.integers(0, 2))
        stream = int(rng.integers(0, 2 ** 63))
        a, b = kq_hip.rng_seed(seed, stream), kq_oracle.rng_seed(seed, stream)
        for _ in range(50):
            assert kq_hip.rng_next(a) == kq_oracle.rng_next(b)
        assert (a.state, a.draws, a.integrity) == (b.state, b.draws, b.integrity)


def test_rng_record_checks():
    L = kq_hip.lib()
    st = kq_hip.rng_seed(7, kq_hip.SAMPLING_DEFAULT_STREAM)
    assert status_of(L.kq_hip_sampling_rng_seed, 1, 2 ** 63, C.byref(kq_hip.RngState()))[0] == \
        "INVALID_ARGUMENT"
    assert status_of(L.kq_hip_sampling_rng_seed, 1, 2, None)[0] == "INVALID_ARGUMENT"
    for field, value in (("version", 2), ("reserved", 1), ("increment", 4), ("state", 99),
                         ("integrity", 0)):
        bad = kq_hip.RngState.from_buffer_copy(st)
        setattr(bad, field, value)
        w = C.c_uint32(1234)
        name, d = status_of(L.kq_hip_sampling_rng_next_u32, C.byref(bad), C.byref(w))
        assert name == "INVALID_RNG_STATE" and w.value == 1234, field
        assert status_of(L.kq_hip_sampling_rng_reset, C.byref(bad))[0] == "INVALID_RNG_STATE"
        out = kq_hip.RngState()
        assert status_of(L.kq_hip_sampling_rng_snapshot, C.byref(bad), C.byref(out))[0] == \
            "INVALID_RNG_STATE"
    # the draw counter at its maximum: the state does not move
    top = kq_hip.RngState.from_buffer_copy(st)
    top.draws = 2 ** 64 - 1
    top.integrity = integrity(top)
    before = bytes(top)
    assert status_of(L.kq_hip_sampling_rng_next_u32, C.byref(top), C.byref(C.c_uint32()))[0] == \
        "ARITHMETIC_OVERFLOW"
    assert bytes(top) == before
    # reset returns to the seeded record, snapshot/import copy it
    for _ in range(5):
        kq_hip.rng_next(st)
    snap = kq_hip.RngState()
    assert status_of(L.kq_hip_sampling_rng_snapshot, C.byref(st), C.byref(snap))[0] == "OK"
    assert bytes(snap) == bytes(st)
    imp = kq_hip.RngState()
    assert status_of(L.kq_hip_sampling_rng_import, C.byref(snap), C.byref(imp))[0] == "OK"
    assert kq_hip.rng_next(imp) == kq_hip.rng_next(st)
    assert status_of(L.kq_hip_sampling_rng_reset, C.byref(st))[0] == "OK"
    assert bytes(st) == bytes(kq_hip.rng_seed(7, kq_hip.SAMPLING_DEFAULT_STREAM))


def test_default_policy():
    p = kq_hip.default_policy()
    assert (p.version, p.flags, p.top_k, list(p.reserved)) == (1, 0, 20, [0, 0, 0])
    assert p.temperature == 1.0 and p.top_p == np.float32(0.95)


BAD_POLICIES = [dict(version=2), dict(flags=1), dict(reserved=(0, 1, 0)),
                dict(temperature=0.0), dict(temperature=-1.0), dict(temperature=float("inf")),
                dict(temperature=float("nan")), dict(top_p=-0.01), dict(top_p=1.01),
                dict(top_p=float("nan")), dict(top_k=248321)]


@pytest.mark.parametrize("bad", BAD_POLICIES, ids=lambda b: "-".join(f"{k}" for k in b))
def test_config_open_rejects_policy(bad):
    L = kq_hip.lib()
    p = kq_hip.sampling_policy(**bad)
    h = C.c_void_p(0x1234)
    name, d = status_of(L.kq_hip_sampling_config_open_qwen38, C.byref(p), C.byref(h))
    assert name == "INCOMPATIBLE_SAMPLING" and h.value is None, d.message


def test_config_open_argument_checks():
    L = kq_hip.lib()
    p = kq_hip.default_policy()
    assert status_of(L.kq_hip_sampling_config_open_qwen38, C.byref(p), None)[0] == \
        "INVALID_ARGUMENT"
    h = C.c_void_p()
    assert status_of(L.kq_hip_sampling_config_open_qwen38, None, C.byref(h))[0] == \
        "INCOMPATIBLE_SAMPLING"
    for vocab, canon, want in ((0, 0, "INVALID_ARGUMENT"), (10, 11, "INVALID_ARGUMENT"),
                               (10, 0, "INVALID_ARGUMENT"), (2 ** 24 + 1, 5, "LIMIT_EXCEEDED")):
        assert status_of(L.kq_hip_sampling_config_open, C.byref(p), vocab, canon,
                         C.byref(h))[0] == want
    # top_k is checked against the configured vocabulary
    p.top_k = 11
    assert status_of(L.kq_hip_sampling_config_open, C.byref(p), 10, 10, C.byref(h))[0] == \
        "INCOMPATIBLE_SAMPLING"
    # invalid handles report nothing
    assert L.kq_hip_sampling_required_scratch_bytes(None) == 0
    assert L.kq_hip_sampling_config_vocabulary_size(None) == 0
    assert L.kq_hip_sampling_config_owned_bytes(None) == 0
    L.kq_hip_sampling_config_close(None)
