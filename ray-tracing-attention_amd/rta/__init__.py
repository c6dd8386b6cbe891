"""MI355X (gfx950) detector path of Ray Tracing Attention.

librta.so holds the HIP kernels behind a C ABI (include/rta.h); this package is
its host-side mirror: ctypes binding (_lib), torch-tensor operators (ops),
seeded synthetic superblocks (synth) and the diagnostic runtime that mirrors the
reference's ResidentRuntime.mlp / .vocabulary / .attention operators (runtime).
"""
from ._lib import BF16, F16, F32, Q4_K, Q6_K, RtaError, load  # noqa: F401

__all__ = ["BF16", "F16", "F32", "Q4_K", "Q6_K", "RtaError", "load"]
