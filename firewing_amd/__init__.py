"""MI355X-native sparse-MoE block hot path of Firewing (router top-k, routed and
shared SwiGLU experts, ordered top-k mixture) behind a C ABI.

The HIP library is libfirewing_hip_moe.so (include/firewing_hip_moe.h); the
Python mirror of the reference's entry points is firewing_amd.hip_moe.
"""
__all__ = ["hip_moe", "build"]
