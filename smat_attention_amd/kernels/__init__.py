"""HIP kernels of the SMat schedule and their Python bindings.

``hip_fwd`` is the drop-in for the reference's ``smat.kernels.triton_fwd``
(the module ``smat.attention`` imports as ``_tri``); ``triton_fwd`` is kept as
an alias so code written against the reference's module path keeps working.
"""
from . import hip_fwd  # noqa: F401
from . import hip_bwd  # noqa: F401
