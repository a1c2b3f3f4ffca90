import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP library)")


@pytest.fixture(scope="session")
def enc():
    """One okf context on cuda:0 for the whole GPU session."""
    import torch
    import chatokf_amd as ok

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    torch.cuda.init()
    e = ok.Enc(0)
    yield e
    e.close()
