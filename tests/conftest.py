import importlib.util
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_DIR = os.path.join(ROOT, "embeddinggemma2-amdkfd_amd")
sys.path.insert(0, os.path.join(ROOT, "oracle"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def load_package():
    """Imports the package's Python binding (the directory name is not a
    valid module name, so it is loaded from its path)."""
    if "eg2hip" in sys.modules:
        return sys.modules["eg2hip"]
    spec = importlib.util.spec_from_file_location("eg2hip", os.path.join(PKG_DIR, "eg2hip.py"))
    mod = importlib.util.module_from_spec(spec)
    sys.modules["eg2hip"] = mod
    spec.loader.exec_module(mod)
    return mod


@pytest.fixture(scope="session")
def eg2():
    return load_package()


@pytest.fixture(scope="session")
def gpu(eg2):
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a visible GPU")
    err = __import__("ctypes").create_string_buffer(256)
    if eg2.lib().eg2_hip_device_check(err, 256) != 0:
        pytest.fail("device check failed: " + err.value.decode())
    return torch.device("cuda:0")


@pytest.fixture(scope="session")
def full_model(eg2, tmp_path_factory):
    """The 24-layer model of the 16x128 benchmark wave: seed 0, full
    attention with RoPE base 1e4, dense head (written once per session)."""
    path = str(tmp_path_factory.mktemp("full") / "full.gguf")
    eg2.synth_gguf(path, seed=0, n_layer=24, dense_head=True, sliding_window=0, rope_base_full=1e4,
                   rope_base_swa=1e4, threads=16)
    return path
