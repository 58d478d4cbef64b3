"""Shared test setup: import paths, the `gpu` marker, small synthetic models.

`-m "not gpu"` runs on any host (oracle vs golden vectors, host logic, the C ABI's argument
checks); `-m gpu` needs an MI355X and compares the HIP path with the oracle.
"""

import os
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
PKG = ROOT / "pico-engine_amd"
for p in (str(ROOT), str(PKG)):
    if p not in sys.path:
        sys.path.insert(0, p)

GOLDEN = ROOT / "tests" / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (MI355X) and the built libpico_hip.so")
    config.addinivalue_line("markers", "slow: runs a full-size model (minutes)")


def gpu_available() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:  # noqa: BLE001
        return False


def pytest_collection_modifyitems(config, items):
    if gpu_available():
        return
    skip = pytest.mark.skip(reason="no GPU on this host")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def oracle_clib():
    """ctypes handle of oracle/_build/liboracle_dequant.so (built on demand with make)."""
    import ctypes
    so = ROOT / "oracle" / "_build" / "liboracle_dequant.so"
    if not so.exists():
        subprocess.run(["make", "-C", str(ROOT / "oracle")], check=True, capture_output=True)
    lib = ctypes.CDLL(str(so))
    lib.oracle_dequantize.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p]
    lib.oracle_dequantize.restype = ctypes.c_int
    lib.oracle_half_to_float.argtypes = [ctypes.c_uint16]
    lib.oracle_half_to_float.restype = ctypes.c_float
    return lib


@pytest.fixture(scope="session")
def model_dir(tmp_path_factory):
    d = os.environ.get("PICO_HIP_CACHE")
    if not d:
        return tmp_path_factory.mktemp("models")
    Path(d).mkdir(parents=True, exist_ok=True)
    return Path(d)


@pytest.fixture(scope="session")
def tiny_model(model_dir):
    """A 2-layer model of the 0.5B family (Q5_0/Q8_0/Q6_K/Q4_K mix), built once per session."""
    from pico_hip import synth
    arch = synth.tiny_arch(n_layers=2, hidden=256, n_head=4, n_kv=2, head_dim=64, ffn=512, vocab=1024)
    path = model_dir / "tiny-2l.gguf"
    if not path.exists():
        synth.build(path, arch, seed=7)
    return path
