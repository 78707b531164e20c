import os
import sys

import pytest

# The HIP runtime's graph launch path as the benchmark runs it (bench.py):
# kernel nodes launched like eager kernels instead of as pre-recorded AQL
# packets.  It must be set before the runtime initializes, i.e. before any
# test imports torch; the graph tests then check replays bitwise against the
# eager calls under the setting the benchmark measures.
os.environ.setdefault("DEBUG_CLR_GRAPH_PACKET_CAPTURE", "0")

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X); runs the parity tests through the C ABI")


@pytest.fixture(scope="session")
def gpu():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    import kvbridge_amd

    kvbridge_amd.load()  # fails loudly if the library was not built
    return torch.device("cuda:0")
