import importlib
import os
import shutil
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "oracle"), os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device) to run")


@pytest.fixture(scope="session")
def orc():
    import oracle

    oracle.lib()
    return oracle


def _random_weights(tmp_path_factory, env, preset, name, need_gb):
    """Seeded random-init weights (seed 0, N(0, 0.02)) written once per session,
    or the file named by the environment variable `env`."""
    path = os.environ.get(env)
    if path:
        return path
    myos = importlib.import_module("an-operating-system-for-ai-models-and-tensor-inference_amd")
    d = tmp_path_factory.mktemp("weights")
    free = shutil.disk_usage(str(d)).free / 1e9
    if free < need_gb:
        pytest.skip(f"{free:.0f} GB free under {d}; the {name} weights need {need_gb} GB")
    path = str(d / f"{name}_seed0.safetensors")
    print(f"writing {name} random-init weights to {path}", flush=True)
    myos.write_random_qwen25(path, myos.preset(preset), seed=0, std=0.02,
                             threads=min(16, os.cpu_count() or 1))
    return path


@pytest.fixture(scope="session")
def qwen15_path(tmp_path_factory):
    myos = importlib.import_module("an-operating-system-for-ai-models-and-tensor-inference_amd")
    return _random_weights(tmp_path_factory, "MYOS_TEST_WEIGHTS_1_5B",
                           myos.SHAPE_QWEN25_1_5B, "qwen25_1_5b", 4)


@pytest.fixture(scope="session")
def qwen7b_path(tmp_path_factory):
    myos = importlib.import_module("an-operating-system-for-ai-models-and-tensor-inference_amd")
    return _random_weights(tmp_path_factory, "MYOS_TEST_WEIGHTS_7B",
                           myos.SHAPE_QWEN25_7B, "qwen25_7b", 17)
