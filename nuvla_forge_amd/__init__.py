"""nuvla_forge_amd: MI355X-native fused adaLN-RMSNorm, SwiGLU and chunked
cross entropy behind the ``nuvla_forge.kernels`` API.

Layout:
  csrc/      HIP kernels for gfx950 and the C ABI (include/nuvla_forge_hip.h)
  build.py   hipcc build of libnf_hip.so, in-tree
  _lib.py    ctypes binding of the C ABI
  kernels/   the drop-in Python package (autograd Functions, public ops)
"""

__version__ = "0.1.0"
