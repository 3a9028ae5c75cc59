"""SMat attention's chunkwise schedule on AMD Instinct MI355X (gfx950).

``mask``       host geometry of M^(d) (the reference's src/smat/mask.py API)
``attention``  the schedule on the GPU (the reference's src/smat/attention.py API)
``kernels``    the HIP kernels behind the ``kernels/`` dispatch (libsmat_hip.so)
"""
from . import mask  # noqa: F401

__version__ = "0.1.0"


def __getattr__(name):
    # attention/kernels import torch; load them on first use
    if name in ("attention", "kernels"):
        import importlib
        return importlib.import_module(f"{__name__}.{name}")
    raise AttributeError(name)
