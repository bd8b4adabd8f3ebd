"""tallymap_amd: an MI355X-native (gfx950, HIP) kernel backend for tallymap-style `vmap` programs.

An item function of ONE item (its own while loop, its own jax.random draws, results added into write-only
tallies) is traced into a jaxpr-shaped program, lowered to HIP, compiled with hipRTC for gfx950 and launched as
one persistent wave64 kernel through the C-ABI library libtallymap_rocm.so.  Reverse-mode gradients run the
replay adjoint (a step-scheduled replay over a tape in HBM, or an ordinary item program when no loop carry needs a
reverse sweep) through the same path; forward-mode derivatives (jvp, jacfwd) run one fused tangent kernel.  Items
that spawn children (Queue) run generation by generation, one launch of the same kernel per generation.
"""
from . import lax, numpy, random
from ._api import (STATS, Queue, Records, Result, Sum, TallyError, UnsupportedError, grad, jacfwd, jvp,
                   value_and_grad, vjp, vmap)
from ._tally import Tally

__version__ = "0.1.0"
__all__ = ["vmap", "vjp", "grad", "value_and_grad", "jvp", "jacfwd", "Sum", "Queue", "Records", "Result", "STATS", "Tally", "TallyError", "UnsupportedError", "lax", "numpy", "random"]
