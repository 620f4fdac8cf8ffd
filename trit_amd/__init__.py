"""trit_amd: Trit's decoder token loop on MI355X (gfx950).

The product is libtrit_hip.so (hand-written HIP kernels behind the C ABI
of include/trit_hip.h). `trit_amd.hip` is a ctypes driver of that ABI for
Python callers and tests; it fails loudly when the library is missing.
"""

__all__ = ["hip", "synth"]
