import json
import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
PKG = ROOT / "kestrel-q_amd"
GOLDEN = Path(__file__).resolve().parent / "golden"

for p in (ROOT / "oracle", PKG):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) device")


def load_golden(name: str) -> dict:
    return json.loads((GOLDEN / name).read_text())


def hex_le_f32(s: str):
    import numpy as np
    return np.frombuffer(bytes.fromhex(s), dtype="<f4").astype(np.float32)


def bits_f32(hexes):
    """List of big-endian-written f32 bit patterns ('3f800000') -> array."""
    import numpy as np
    return np.array([int(h, 16) for h in hexes], dtype=np.uint32).view(np.float32)


def ulp_distance(a, b):
    import numpy as np
    a = np.asarray(a, np.float32).view(np.int32).astype(np.int64)
    b = np.asarray(b, np.float32).view(np.int32).astype(np.int64)
    a = np.where(a < 0, -(a & 0x7FFFFFFF), a)
    b = np.where(b < 0, -(b & 0x7FFFFFFF), b)
    return np.abs(a - b)


RTOL, ATOL = 1e-3, 1e-4
# One record per assert_close call: test id, what was compared and its
# errors. Written as JSON lines to $KQ_TOL_LOG at the end of the session.
TOL_RECORDS: list = []


# Third stage of assert_close: the error against the binary64 value at most
# this fraction of the element's term magnitude S (tests/exact.py): 2^-23 is
# 2 u (u = 2^-24, binary32's unit roundoff), about 16 times the largest
# ratio measured on the device over the GPU suite (7.5e-9).
COND_TOL = 2.0 ** -23
# Ceiling on the elements one call may pass through the second and third
# stages together, as a fraction of its elements (at least FALLBACK_MIN):
# the fallbacks are for the few elements where the oracle's own binary32
# sum is off, not a second bar for a whole output.
FALLBACK_FRAC = 0.005
FALLBACK_MIN = 4


def assert_close(got, ref, rtol=RTOL, atol=ATOL, exact=None, what="", max_fallback=None,
                 cond_tol=COND_TOL):
    """fp32-accumulated outputs, per element: |got - ref| <= atol OR
    |got - ref| <= rtol * |ref| (the reference's validator rule,
    tools/validate-native-moe.py:186-189, with the contract's 1e-4 absolute
    and 1e-3 relative limits).

    `exact` (optional, tests/exact.py) gives the binary64 value of the same
    equations on the same decoded weights at flat element indices, and
    possibly the magnitude S of the terms each element is summed from.
    Elements beyond the bar against `ref` are checked again:
      2. within the same bar of the exact value: the reference's own
         left-to-right binary32 sum is off there (a 2048-term row whose
         partial sums reach ~100 rounds each step by ~1e-6);
      3. otherwise, where S is given: |got - exact| <= 2^-23 * S. At these
         elements the output is a near-cancellation of terms many times its
         size, where no binary32 evaluation meets the bar (the reference's
         own error against the exact value is recorded beside the device's).
         Binary32 rounding in any order stays near u * S (u = 2^-24); a
         wrong, missing or transposed term moves the element by about one
         term, above 1e-4 * S.
    `cond_tol` replaces COND_TOL where a test states why its bar differs.
    At most `max_fallback` elements (default: FALLBACK_FRAC of the elements,
    at least FALLBACK_MIN) may take stages 2 and 3 together.
    Counts and the largest ratios of each stage are recorded."""
    import numpy as np
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    assert np.isfinite(got).all()
    err = np.abs(got - ref)
    ok = (err <= atol) | (err <= rtol * np.abs(ref))
    rel = np.where(err > atol, err / np.maximum(np.abs(ref), np.finfo(np.float64).tiny), 0.0)
    rec = {"test": os.environ.get("PYTEST_CURRENT_TEST", "").split(" ")[0], "what": what,
           "n": int(err.size), "max_abs": float(err.max(initial=0.0)),
           "max_rel_beyond_abs": float(rel.max(initial=0.0)),
           "max_abs_ref": float(np.abs(ref).max(initial=0.0)),
           "beyond_bar_vs_ref": int((~ok).sum())}
    TOL_RECORDS.append(rec)
    if ok.all():
        return rec
    bad = np.flatnonzero(~ok)
    ceiling = max_fallback if max_fallback is not None else max(
        FALLBACK_MIN, int(np.ceil(FALLBACK_FRAC * err.size)))
    rec["fallback_ceiling"] = int(ceiling)
    if bad.size > ceiling:
        i = bad[:5]
        raise AssertionError(
            f"{bad.size} elements beyond 1e-4 abs / 1e-3 rel of the reference, more than the "
            f"{ceiling} the exact-value fallbacks may take; first {i.tolist()}: got "
            f"{got.flat[i]}, ref {ref.flat[i]}, err {err.flat[i]}")
    if exact is None:
        i = bad[:5]
        raise AssertionError(
            f"{bad.size} elements beyond 1e-4 abs / 1e-3 rel, first {i.tolist()}: got "
            f"{got.flat[i]}, ref {ref.flat[i]}, err {err.flat[i]}")
    ex = np.asarray(exact(bad), np.float64)
    eg = np.abs(got.flat[bad] - ex)
    er = np.abs(ref.flat[bad] - ex)
    ok2 = (eg <= atol) | (eg <= rtol * np.abs(ex))
    rec.update({"within_bar_of_exact": int(ok2.sum()),
                "max_err_vs_exact_stage2": float(eg[ok2].max(initial=0.0)),
                "ref_err_vs_exact_stage2": float(er[ok2].max(initial=0.0))})
    if ok2.all():
        return rec
    b3 = bad[~ok2]
    scale = getattr(exact, "scale", None)
    if scale is None:
        raise AssertionError(
            f"{b3.size} elements beyond the bar against both the reference and the exact "
            f"value, first {b3[:5].tolist()}: got {got.flat[b3[:5]]}, ref {ref.flat[b3[:5]]}, "
            f"exact {ex[~ok2][:5]}")
    S3 = np.asarray(scale(b3), np.float64)
    r3 = eg[~ok2] / S3
    rec.update({"cancellation_elements": int(b3.size),
                "max_err_over_S": float(r3.max()),
                "ref_max_err_over_S": float((er[~ok2] / S3).max()),
                "max_err_vs_exact_stage3": float(eg[~ok2].max()),
                "ref_err_vs_exact_stage3": float(er[~ok2].max()),
                "min_S_over_abs_exact": float((S3 / np.maximum(np.abs(ex[~ok2]), 1e-300)).min())})
    rec["cond_tol"] = float(cond_tol)
    if not (r3 <= cond_tol).all():
        j = np.flatnonzero(r3 > cond_tol)[:5]
        raise AssertionError(
            f"{int((r3 > cond_tol).sum())} elements beyond the bar against the reference and "
            f"the exact value, and beyond {cond_tol:.3g} of their term magnitude: indices "
            f"{b3[j].tolist()}, got {got.flat[b3[j]]}, exact {ex[~ok2][j]}, S {S3[j]}")
    return rec


def record(what: str, values: dict) -> None:
    """A measured figure of a test (counts, rates) for the same log."""
    TOL_RECORDS.append({"test": os.environ.get("PYTEST_CURRENT_TEST", "").split(" ")[0],
                        "what": what, **values})


def pytest_sessionfinish(session, exitstatus):
    path = os.environ.get("KQ_TOL_LOG")
    if path and TOL_RECORDS:
        with open(path, "a") as f:
            for r in TOL_RECORDS:
                f.write(json.dumps(r) + "\n")


@pytest.fixture(scope="session")
def oracle():
    import kq_oracle
    return kq_oracle


def oracle_threads() -> int:
    return int(os.environ.get("KQ_ORACLE_THREADS", min(16, os.cpu_count() or 1)))
