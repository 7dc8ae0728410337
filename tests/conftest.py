"""Shared fixtures. GPU tests carry @pytest.mark.gpu; everything else runs on CPU."""
from __future__ import annotations

import json
import pathlib
import sys

import numpy as np
import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
GOLDEN = ROOT / "tests" / "golden"
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) device")


def _ensure_built():
    lib = ROOT / "modelsharp_amd" / "lib" / "libms_hip_nbits.so"
    orc = ROOT / "oracle" / "liboracle_nbits.so"
    if not lib.is_file() or not orc.is_file():
        import __graft_entry__
        __graft_entry__.build()


_ensure_built()


@pytest.fixture(scope="session")
def kat_cases():
    return json.loads((GOLDEN / "kat_vectors.json").read_text())["cases"]


@pytest.fixture(scope="session")
def ref_vectors():
    with np.load(GOLDEN / "ref_qgemm_vectors.npz") as z:
        data = {k: z[k] for k in z.files}
    groups: dict[str, dict] = {}
    for k, v in data.items():
        g, field = k.split("/")
        groups.setdefault(g, {})[field] = v
    return groups


@pytest.fixture(scope="session")
def gpu():
    """The library, with a usable gfx950 device (GPU tests only)."""
    from modelsharp_amd import native
    lib = native.load()
    if not native.available():
        pytest.fail("gpu test on a host without a gfx950 device: " + native.last_error())
    return lib


def kat_arrays(case):
    a = np.array(case["a"], np.float32).reshape(case["a_shape"])
    b = np.array(case["b"], np.uint8).reshape(case["b_shape"])
    s = np.array(case["scales"], np.float32)
    zp = None
    if case["zp"] is not None:
        zp = np.array(case["zp"], np.uint8 if case["zp_dtype"] == "uint8" else np.float32)
    y = np.array(case["y"], np.float32).reshape(case["y_shape"])
    return a, b, s, zp, y


@pytest.fixture(scope="session")
def w4a8_vectors():
    with np.load(GOLDEN / "ref_w4a8_vectors.npz") as z:
        data = {k: z[k] for k in z.files}
    groups: dict[str, dict] = {}
    for k, v in data.items():
        g, field = k.split("/")
        groups.setdefault(g, {})[field] = v
    return groups
