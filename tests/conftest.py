"""Shared fixtures.  `-m "not gpu"` runs the oracle, host logic and C-ABI checks on the CPU;
`-m gpu` runs the HIP parity tests (they call the engine through the C ABI in libsdhip.so)."""
import importlib.util
import os
import sys
import tempfile
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
PKG_DIR = ROOT / "strands-decider-rs_amd"
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def load_pkg():
    """The package directory has a hyphenated name, so it is imported by path as `sdamd`."""
    if "sdamd" in sys.modules:
        return sys.modules["sdamd"]
    spec = importlib.util.spec_from_file_location("sdamd", PKG_DIR / "__init__.py",
                                                  submodule_search_locations=[str(PKG_DIR)])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["sdamd"] = mod
    spec.loader.exec_module(mod)
    return mod


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the HIP engine)")


@pytest.fixture(scope="session")
def sdamd():
    return load_pkg()


@pytest.fixture(scope="session")
def synth(sdamd):
    import sdamd.synth as s
    return s


@pytest.fixture(scope="session")
def oracle():
    from oracle import torso
    torso.lib()  # raises if liboracle.so is not built
    return torso


def _model_dir(name):
    base = os.environ.get("SD_TEST_MODELS") or os.path.join(tempfile.gettempdir(), "sd_test_models")
    return os.path.join(base, name)


@pytest.fixture(scope="session")
def tiny_model(synth):
    """A small hybrid (8 layers, hidden 512) in the reference's model-directory format."""
    return synth.write_model(_model_dir("tiny"), synth.CONFIG_TINY, vocab=4096, seed=1)


@pytest.fixture(scope="session")
def model_2b(synth):
    """The benchmark's 2B hybrid (24 layers, hidden 2048, vocab 151936), seeded random weights."""
    return synth.write_model(_model_dir("2b"), synth.CONFIG_2B, vocab=synth.VOCAB_2B, seed=0)


def f16_ulp(x):
    """Spacing of float16 at |x| (subnormal spacing below 2^-14)."""
    a = np.abs(np.asarray(x, np.float32)).astype(np.float16)
    return np.spacing(a).astype(np.float32)
