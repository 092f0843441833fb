import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

# One HIP runtime per process: torch brings its own libamdhip64, and a process
# that loads libhip_bridge.so (system ROCm) before importing torch can crash in
# torch's import. Import torch first, before any test can load the library.
try:
    import torch  # noqa: F401
except ImportError:  # pragma: no cover - torch is optional for the CPU tests
    pass


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (run with -m gpu)")


@pytest.fixture(scope="session")
def gpu():
    """torch (device memory and streams only) + one hip_bridge context bound to
    torch's current stream, so torch copies and library kernels are ordered."""
    import torch  # import before the library: one HIP runtime per process
    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a visible GPU")
    from rustane_amd import hip_bridge as hb
    # A dedicated (default-priority) stream for torch and the library alike.
    stream = torch.cuda.Stream()
    torch.cuda.set_stream(stream)
    ctx = hb.Context(0)
    ctx.set_stream(stream.cuda_stream)
    yield ctx
    torch.cuda.synchronize()
    ctx.close()
