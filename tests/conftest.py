import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "hilbert-pruned-8b_amd")
for p in (PKG, os.path.join(ROOT, "oracle"), os.path.join(ROOT, "tests", "golden")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU (runs on the GPU box)")


@pytest.fixture(scope="session")
def oracle():
    import oracle as o
    return o.Oracle()


@pytest.fixture(scope="session")
def reference():
    import oracle as o
    if not os.path.exists(o.REF_PATH):
        pytest.skip("oracle/_ref/libref.so not built (needs /root/reference)")
    return o.Reference()


@pytest.fixture(scope="session")
def hqlib():
    """The product library on a GPU: loads libhq.so and selects device 0 (gfx950 checked)."""
    import hq
    hq.load()
    print(f"[gpu] device: {hq.device_name(0)}", flush=True)
    hq.device_init(0)
    return hq


def rel_l2(got, ref):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.linalg.norm(got - ref) / max(np.linalg.norm(ref), 1e-30))


def max_abs(got, ref):
    return float(np.max(np.abs(np.asarray(got, np.float64) - np.asarray(ref, np.float64)))) if np.size(ref) else 0.0


def same_bits_nan_aware(a, b):
    """float32 arrays equal bit for bit, except that any NaN matches any NaN."""
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    na, nb = np.isnan(a), np.isnan(b)
    return bool(np.array_equal(na, nb) and np.array_equal(a[~na].view(np.uint32), b[~nb].view(np.uint32)))
