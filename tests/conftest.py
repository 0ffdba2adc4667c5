import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "shannon-prime-system_amd"))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, os.path.join(ROOT, "tests"))


def pytest_configure(config):
    # the oracle's row-parallel loops (bit-identical for any count): the host's
    # cores, at most 16
    try:
        import orc
        orc.lib().orc_set_threads(min(16, os.cpu_count() or 1))
    except Exception:
        pass
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP backend)")
    config.addinivalue_line("markers", "slow: long-running parity case")


@pytest.fixture(scope="session")
def tmpdir_models(tmp_path_factory):
    return tmp_path_factory.mktemp("models")
