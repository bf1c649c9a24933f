"""MI355X (gfx950) rebuild of the REAX engine's fused attention path.

The product is the pair of C-ABI libraries in lib/ (libreax_howu.so, libreax_fmha_post.so). This package holds
their ctypes binding (abi), torch-facing wrappers (ops, imported on demand: `from reax_fmha import ops`) and the
benchmark configurations (workloads).
"""
from . import abi, workloads  # noqa: F401
