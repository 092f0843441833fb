"""MI355X (gfx950) implementation of rustane's transformer forward path and
single-token decode loop, behind the C ABI of libhip_bridge.so.

  hip_bridge  ctypes binding of include/hip_bridge.h (the `hip-bridge` crate's role)
  engine      rustane's engine API (ModelConfig, ModelWeights, forward_ws, ...)
"""
__all__ = ["hip_bridge", "engine"]
