"""MI355X (gfx950) fused kernels for VLA-style driving models.

Drop-in for ``nuvla_forge.kernels`` (reference ``nuvla_forge/kernels/__init__.py:8-18``):
the same three ops and the same ``HAS_TRITON`` flag, backed by hand-written HIP
kernels in ``libnf_hip.so`` instead of Triton; plus ``fused_gate_up_swiglu``,
the SwiGLU fused into its gate/up projection GEMM.
"""

from .adaln_rmsnorm import fused_adaln_residual_rmsnorm
from .chunked_ce import chunked_cross_entropy
from .swiglu import fused_gate_up_swiglu, fused_swiglu
from .utils import HAS_HIP, HAS_TRITON

__all__ = [
    "HAS_HIP",
    "HAS_TRITON",
    "chunked_cross_entropy",
    "fused_adaln_residual_rmsnorm",
    "fused_gate_up_swiglu",
    "fused_swiglu",
]
