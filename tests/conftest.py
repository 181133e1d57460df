"""Test configuration: the ``gpu`` marker, import paths and shared models.

``-m "not gpu"`` runs the CPU suite (oracle against golden vectors and closed
forms, host logic, the C ABI's exports); ``-m gpu`` runs the parity tests of
the HIP path against the CPU oracle on one MI355X.
"""

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "symmetrix-xl_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device) to run")


MODEL_DIR = os.environ.get("SYMMETRIX_MODEL_CACHE", "/tmp/symmetrix_models")


@pytest.fixture(scope="session")
def tiny_model_path():
    from symmetrix import random_model
    return random_model.cached_model("tiny", directory=MODEL_DIR)


@pytest.fixture(scope="session")
def medium_model_path():
    from symmetrix import random_model
    return random_model.cached_model("medium", directory=MODEL_DIR)


@pytest.fixture(scope="session")
def wide_model_path():
    from symmetrix import random_model
    return random_model.cached_model("wide", directory=MODEL_DIR)


@pytest.fixture(scope="session")
def tiny_scaled_model_path():
    from symmetrix import random_model
    return random_model.cached_model("tiny_scaled", directory=MODEL_DIR)


@pytest.fixture(scope="session")
def tiny_zbl_model_path():
    from symmetrix import random_model
    return random_model.cached_model("tiny_zbl", directory=MODEL_DIR)


@pytest.fixture(scope="session")
def tiny_heads_model_path():
    from symmetrix import random_model
    return random_model.cached_model("tiny_heads", directory=MODEL_DIR)


@pytest.fixture(scope="session")
def tiny_plu_model_path():
    from symmetrix import random_model
    return random_model.cached_model("tiny_plu", directory=MODEL_DIR)


@pytest.fixture(scope="session")
def tiny_residual_model_path():
    from symmetrix import random_model
    return random_model.cached_model("tiny_residual", directory=MODEL_DIR)


@pytest.fixture(scope="session")
def tiny_single_model_path():
    from symmetrix import random_model
    return random_model.cached_model("tiny_single", directory=MODEL_DIR)


@pytest.fixture(scope="session")
def tiny_single_residual_model_path():
    from symmetrix import random_model
    return random_model.cached_model("tiny_single_residual", directory=MODEL_DIR)


@pytest.fixture(scope="session")
def tiny_field_model_path():
    from symmetrix import random_model
    return random_model.cached_model("tiny_field", directory=MODEL_DIR)


@pytest.fixture(scope="session")
def tiny_field_scaled_model_path():
    from symmetrix import random_model
    return random_model.cached_model("tiny_field_scaled", directory=MODEL_DIR)


@pytest.fixture(scope="session")
def field_l2_model_path():
    from symmetrix import random_model
    return random_model.cached_model("field_l2", directory=MODEL_DIR)


@pytest.fixture(scope="session")
def medium_single_model_path():
    from symmetrix import random_model
    return random_model.cached_model("medium_single", directory=MODEL_DIR)


@pytest.fixture(scope="session")
def tiny_agnesi_model_path():
    from symmetrix import random_model
    return random_model.cached_model("tiny_agnesi", directory=MODEL_DIR)
