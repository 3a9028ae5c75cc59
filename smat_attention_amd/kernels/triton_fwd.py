"""Alias of :mod:`smat_attention_amd.kernels.hip_fwd` under the reference's
module name (src/smat/kernels/triton_fwd.py), for code that imports it by
that path.  Nothing here uses Triton."""
from .hip_fwd import *  # noqa: F401,F403
from .hip_fwd import available, chunk_local, incidence, pool, pool_ok  # noqa: F401
