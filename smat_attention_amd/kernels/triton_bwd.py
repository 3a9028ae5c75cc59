"""Alias of :mod:`smat_attention_amd.kernels.hip_bwd` under the reference's
module name (src/smat/kernels/triton_bwd.py).  Nothing here uses Triton."""
from .hip_bwd import *  # noqa: F401,F403
from .hip_bwd import patch, unpatch  # noqa: F401
