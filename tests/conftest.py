"""Shared fixtures.  CPU tests check the oracle (against base2.py's golden vectors and closed forms) and the host
logic; tests marked gpu call the HIP library through its C ABI and compare with the oracle."""
from __future__ import annotations

import importlib.util
import json
import os
import sys

import numpy as np
import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if REPO not in sys.path:
    sys.path.insert(0, REPO)

# torch's bundled HIP runtime has the soname the library links (libamdhip64.so.7): loaded first, it is the one
# runtime of this process, so the library and torch's GPU buffers share it
try:
    import torch  # noqa: F401
except ImportError:
    pass


def load_sm():
    if "streaming_machine_amd" in sys.modules:
        return sys.modules["streaming_machine_amd"]
    root = os.path.join(REPO, "streaming-machine_amd")
    spec = importlib.util.spec_from_file_location("streaming_machine_amd", os.path.join(root, "__init__.py"),
                                                  submodule_search_locations=[root])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["streaming_machine_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (calls the HIP library)")


@pytest.fixture(scope="session")
def sm():
    return load_sm()


@pytest.fixture(scope="session")
def golden():
    with open(os.path.join(REPO, "tests", "golden", "base2_golden.json")) as f:
        return json.load(f)


@pytest.fixture(scope="session")
def small_npz(sm):
    return sm.convert(sm.random_gpt2(seed=0, vocab=1000, n_ctx=64))


@pytest.fixture(scope="session")
def full_npz(sm):
    return sm.convert(sm.random_gpt2(seed=0, vocab=50257, n_ctx=1024))


@pytest.fixture(scope="session")
def small_dir(sm, small_npz, tmp_path_factory):
    return sm.layout(small_npz, str(tmp_path_factory.mktemp("small_layout")))


@pytest.fixture(scope="session")
def full_dir(sm, full_npz, tmp_path_factory):
    return sm.layout(full_npz, str(tmp_path_factory.mktemp("full_layout")))


@pytest.fixture(scope="session")
def small_oracle(small_npz):
    import oracle
    return oracle.Oracle(small_npz)


@pytest.fixture(scope="session")
def full_oracle(full_npz):
    import oracle
    return oracle.Oracle(full_npz)


@pytest.fixture(scope="session")
def pgolden():
    with open(os.path.join(REPO, "tests", "golden", "pythia_golden.json")) as f:
        return json.load(f)


@pytest.fixture(scope="session")
def py_small_npz(sm):
    sd, cfg = sm.pythia.random_pythia(seed=5, vocab=1000)
    return sm.pythia.convert_pythia(sd, cfg)


@pytest.fixture(scope="session")
def py_full_npz(sm):
    sd, cfg = sm.pythia.random_pythia(seed=5, vocab=50304)
    return sm.pythia.convert_pythia(sd, cfg)


@pytest.fixture(scope="session")
def py_small_dir(sm, py_small_npz, tmp_path_factory):
    return sm.pythia.pythia_layout(py_small_npz, str(tmp_path_factory.mktemp("py_small_layout")))


@pytest.fixture(scope="session")
def py_full_dir(sm, py_full_npz, tmp_path_factory):
    return sm.pythia.pythia_layout(py_full_npz, str(tmp_path_factory.mktemp("py_full_layout")))


@pytest.fixture(scope="session")
def py_small_oracle(py_small_npz):
    from oracle.pythia import PythiaOracle
    return PythiaOracle(py_small_npz)


def golden_case(golden, name):
    for c in golden["cases"]:
        if c["name"] == name:
            return c
    raise KeyError(name)


def h64(a) -> str:
    import hashlib
    return hashlib.sha256(np.ascontiguousarray(np.asarray(a, dtype=np.int64)).tobytes()).hexdigest()


def synth_qkv(seed: int, P: int, std: float) -> np.ndarray:
    """synthetic gauged QKV rows (int64 at 2^-16) for the attention cases of the golden fixture"""
    rng = np.random.default_rng(seed)
    return np.round(rng.standard_normal((P, 2304)) * std * 65536).astype(np.int64)
