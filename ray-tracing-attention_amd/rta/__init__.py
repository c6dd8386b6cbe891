"""MI355X (gfx950) detector path of Ray Tracing Attention.

librta.so holds the HIP kernels behind a C ABI (include/rta.h); this package is
its host-side mirror: the ctypes binding (_lib), torch-tensor operators with the
argument meanings of the reference's ResidentRuntime.mlp / .vocabulary / .attention
(ops), the hybrid decode step and its synthetic weights and state (model), the
exported-asset reader (asset) and seeded synthetic superblocks (synth).  The
reference's stdin/stdout worker protocol is served by lib/rt_optical_resident.
"""
from ._lib import BF16, F16, F32, Q4_K, Q6_K, RtaError, load  # noqa: F401

__all__ = ["BF16", "F16", "F32", "Q4_K", "Q6_K", "RtaError", "load"]
