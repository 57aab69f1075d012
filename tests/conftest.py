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


def assert_close(got, ref, rtol=RTOL, atol=ATOL):
    """fp32-accumulated outputs: |got - ref| <= atol + rtol * max(|ref|, rms),
    rms taken over each output row (last axis). A reordered fp32 sum errs in
    proportion to the size of its terms, not of its result; the row RMS is
    that scale at elements where the terms cancel. One wrong weight or expert
    moves an element by ~rms/sqrt(n), far above rtol * rms."""
    import numpy as np
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    assert np.isfinite(got).all()
    rms = np.sqrt(np.mean(ref * ref, axis=-1, keepdims=True))
    bound = atol + rtol * np.maximum(np.abs(ref), rms)
    err = np.abs(got - ref)
    bad = err > bound
    if bad.any():
        idx = np.argwhere(bad)[:5]
        raise AssertionError(f"{int(bad.sum())} elements beyond tolerance, first {idx.tolist()}: "
                             f"got {got[bad][:5]}, ref {ref[bad][:5]}, max err/bound "
                             f"{float((err / bound).max()):.3g}")


@pytest.fixture(scope="session")
def oracle():
    import kq_oracle
    return kq_oracle


def oracle_threads() -> int:
    return int(os.environ.get("KQ_ORACLE_THREADS", min(16, os.cpu_count() or 1)))
