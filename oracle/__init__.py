"""CPU oracle for rustane's forward path and decode loop — TEST INFRASTRUCTURE.

This package restates the reference's forward arithmetic in fp32 numpy so the
GPU path can be checked against it. It is a checker only: the product
(libhip_bridge.so and rustane_amd/) never imports it. Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg use it.

Pinning (each function's known-answer / property / independent checks) lives in
tests/test_oracle.py; see oracle/forward.py for the per-function reference
citations.
"""
from .forward import *  # noqa: F401,F403
