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


def pytest_terminal_summary(terminalreporter, exitstatus, config):
    """The parity numbers of every full-size comparison that ran (max |dlogit|,
    max relative per-position loss error, top-1 agreement), and the top-1
    agreement pooled over the comparisons with the oracle."""
    from tests._util import PARITY
    if not PARITY:
        return
    tr = terminalreporter
    tr.write_sep("-", "parity (bars: max|dlogit| <= 2e-2, rel dloss <= 1e-3, top-1 >= 99.5%)")
    for r in PARITY:
        rel = "" if r["rel"] is None else f" rel dloss {r['rel']:.2e}"
        tr.write_line(f"{r['label']}: max|dlogit| {r['err']:.2e}{rel} top-1 {r['same']}/{r['n']} "
                      f"= {100.0 * r['same'] / r['n']:.2f}%")
    o = [r for r in PARITY if r["oracle"]]
    if o:
        same, n = sum(r["same"] for r in o), sum(r["n"] for r in o)
        tr.write_line(f"pooled over {len(o)} oracle comparisons: top-1 {same}/{n} = {100.0 * same / n:.2f}%, "
                      f"max|dlogit| {max(r['err'] for r in o):.2e}, max rel dloss "
                      f"{max((r['rel'] for r in o if r['rel'] is not None), default=0.0):.2e}")


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
