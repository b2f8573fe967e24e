"""MI355X (gfx950) full-attention path of the Bonsai runtime.

The product is the HIP library libbonsai_attn.so behind the C ABI of include/bonsai_attn.h; this package holds
its sources (csrc/), its build (build.py) and the ctypes binding (bonsai_attn.py).
"""
from . import bonsai_attn  # noqa: F401
