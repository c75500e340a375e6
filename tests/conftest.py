import json
import os
import sys

import numpy as np
import pytest

# torch ships its own HIP runtime under the same soname as /opt/rocm's; when
# both are used in one process, torch must load first so libbnn_hip.so binds
# to the runtime already present instead of initialising a second one.
try:
    import torch  # noqa: F401
except ImportError:
    pass

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP engine)")


@pytest.fixture(scope="session")
def orc():
    from oracle.oracle import Oracle, build
    build()
    return Oracle()


@pytest.fixture(scope="session")
def ref():
    from oracle.oracle import RefC, ref_available
    if not ref_available():
        pytest.skip("oracle/_ref not built (reference sources absent)")
    return RefC()


@pytest.fixture(scope="session")
def rorc():
    from oracle.oracle import ReactOracle, build
    build()
    return ReactOracle()


@pytest.fixture(scope="session")
def rref():
    from oracle.oracle import RefReact, react_ref_available
    if not react_ref_available():
        pytest.skip("oracle/_ref not built (reference sources absent)")
    return RefReact()


@pytest.fixture(scope="session")
def golden():
    with open(os.path.join(GOLDEN, "golden.json")) as f:
        meta = json.load(f)
    arrays = dict(np.load(os.path.join(GOLDEN, "golden_logits.npz")))
    return meta, arrays


@pytest.fixture
def blob_file(tmp_path):
    """write a BlobV1 to a temp file and return its path"""
    from bnns_to_c_amd import blob

    def make(b, name="m.blob"):
        p = tmp_path / name
        p.write_bytes(blob.to_bytes(b))
        return str(p)
    return make
