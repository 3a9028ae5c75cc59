"""ctypes binding of libsmat_hip.so (the C ABI declared in include/smat_hip.h).

The library is loaded on first use.  A missing or unloadable library raises
:class:`HipUnavailable` -- there is no fallback: the kernels of this package
are the only implementation of its device path.  A nonzero status from any
entry point raises :class:`HipKernelError` carrying the library's message.
"""
from __future__ import annotations

import contextlib
import ctypes
import os
import threading

import torch

_PKG = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
# The package's own build output, and nothing else: no environment variable
# can point the product at another library.
LIB_PATH = os.path.join(_PKG, "libsmat_hip.so")

SMAT_BF16, SMAT_F16, SMAT_F32 = 0, 1, 2
DTYPE_CODE = {torch.bfloat16: SMAT_BF16, torch.float16: SMAT_F16, torch.float32: SMAT_F32}


class HipUnavailable(ImportError):
    """libsmat_hip.so is not built or cannot be loaded."""


class HipKernelError(RuntimeError):
    """An entry point of libsmat_hip.so returned a nonzero status."""

    def __init__(self, func: str, code: int, msg: str):
        super().__init__(f"{func} failed (status {code}): {msg}")
        self.func, self.code = func, code


_i, _i64, _p, _f = ctypes.c_int, ctypes.c_int64, ctypes.c_void_p, ctypes.c_float

# name -> (restype, argtypes); must match include/smat_hip.h
SIGNATURES = {
    "smat_last_error": (ctypes.c_char_p, []),
    "smat_version": (ctypes.c_char_p, []),
    "smat_set_variant": (_i, [_i, _i]),
    "smat_set_stage_events": (_i, [_p, _i]),
    "smat_chunk_local": (_i, [_i, _p, _p, _p, _p, _p, _i64, _i, _i, _i,
                              _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _p]),
    "smat_chunk_states": (_i, [_i, _p, _p, _p, _i, _i, _i, _i, _i, _i64, _i64, _i64, _i64, _p]),
    "smat_segment_scan": (_i, [_p, _p, _i, _i, _i, _i64, _p]),
    "smat_decay_scan": (_i, [_p, _p, _p, _i, _i, _i, _i64, _p]),
    "smat_decay_scan_reverse": (_i, [_p, _p, _p, _i, _i, _i, _i64, _p]),
    "smat_chunk_local_decay": (_i, [_i, _p, _p, _p, _p, _p, _p, _i64, _i, _i, _i,
                                    _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                                    _p]),
    "smat_causal_scan_workspace_bytes": (_i64, [_i, _i, _i, _i, _i]),
    "smat_causal_scan": (_i, [_i, _p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _i, _i,
                              _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                              _i, _p, _i64, _p]),
    "smat_causal_scan_noalloc_max_bytes": (_i64, []),
    "smat_causal_scan_noalloc": (_i, [_i, _p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _i, _i,
                                      _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                                      _i64, _i64, _i, _p]),
    "smat_segment_scan_reverse": (_i, [_p, _p, _i, _i, _i, _i64, _p]),
    "smat_normalise_backward": (_i, [_p, _p, _p, _p, _p, _i, _i, _i, _i64, _i64, _i64, _i64,
                                     _i64, _i64, _i64, _p]),
    "smat_combine_normalise": (_i, [_i, _p, _p, _p, _i, _i, _i, _i, _f, _i64, _i64, _i64, _i64,
                                    _i64, _i64, _p]),
    "smat_combine_normalise_backward": (_i, [_i, _p, _p, _p, _p, _i, _i, _i, _i, _f, _i64, _i64,
                                             _i64, _i64, _i64, _i64, _i64, _i64, _p]),
    "smat_bgemm": (_i, [_i, _i, _p, _p, _p, _i, _i, _i, _i, _i, _i64, _i64, _i64, _i64,
                        _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i, _i, _p]),
    "smat_chunk_backward": (_i, [_i, _i, _p, _p, _p, _p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _i,
                                 _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                                 _i64, _i64, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64,
                                 _i64, _i64, _p]),
    "smat_chunk_dstates": (_i, [_i, _p, _p, _p, _i, _i, _i, _i, _i, _i64, _i64, _i64, _i64,
                                _p]),
    "smat_lr_dphi": (_i, [_i, _p, _p, _p, _i, _i, _i, _i, _i, _i, _i64, _i64, _i64, _i64,
                          _i64, _i, _p]),
    "smat_lr_dfeat": (_i, [_i, _p, _p, _p, _p, _p, _i, _i, _i, _i, _i64, _i64, _i64, _i64,
                           _i64, _p]),
    "smat_pool_backward": (_i, [_i, _p, _p, _p, _p, _p, _i, _i, _i, _i, _i, _i, _i64, _i64,
                                _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i, _p]),
    "smat_cell_read_backward": (_i, [_i, _i, _p, _p, _p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _i, _i,
                                     _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _p]),
    "smat_cell_pool_backward": (_i, [_i, _i, _p, _p, _p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _i, _i,
                                     _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                                     _i64, _p]),
    "smat_featurise_backward_parts": (_i64, [_i, _i]),
    "smat_forward_fused": (_i, [_i, _p, _p, _p, _p, _p, _i, _p, _i, _p, _i, _p, _i, _p, _p,
                                _i, _i, _i, _i, _i, _i, _i, _i64, _i64, _i64, _i64, _i64,
                                _i64, _i64, _i64, _i64, _i64, _p, _i64, _p]),
    "smat_forward_fused_workspace_bytes": (_i64, [_i, _i, _i, _i, _i, _i, _i]),
    "smat_csr_workspace_bytes": (_i64, [_i, _i, _i]),
    "smat_csr_lists": (_i, [_p, _p, _p, _p, _i, _i, _i, _i, _i64, _i64, _p]),
    "smat_featurise_backward": (_i, [_i, _p, _p, _p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _i, _i,
                                     _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _p]),
    "smat_pool_workspace_bytes": (_i64, [_i, _i, _i, _i, _i, _i]),
    "smat_pool": (_i, [_i, _p, _p, _p, _p, _i, _i, _i, _i, _i, _i,
                       _i64, _i64, _i64, _i64, _p, _i64, _p]),
    "smat_incidence": (_i, [_p, _p, _p, _i, _p, _i, _p, _i, _i, _i, _i64, _p]),
    "smat_incidence_plane": (_i, [_p, _p, _p, _i, _p, _i, _i, _i, _i64, _p]),
    "smat_query": (_i, [_i, _p, _p, _p, _i, _i, _i, _i, _i, _i64, _i64, _i64, _i64, _p]),
    "smat_normalise": (_i, [_p, _p, _p, _p, _i, _i, _i, _i,
                            _i64, _i64, _i64, _i64, _i64, _i64, _i64, _p]),
    "smat_forward_workspace_bytes": (_i64, [_i, _i, _i, _i, _i, _i, _i, _i, _i]),
    "smat_forward": (_i, [_i, _p, _p, _p, _p, _i, _p, _i, _p, _i, _p, _p, _p,
                          _i, _i, _i, _i, _i, _i, _i, _i, _i,
                          _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                          _p, _i64, _p]),
    "smat_direct": (_i, [_i, _p, _p, _p, _p, _i, _p, _i, _i, _i, _i, _i, _i64, _i64, _i64, _i64,
                         _p]),
    "smat_featurise": (_i, [_i, _p, _p, _p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _i, _i,
                            _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                            _p]),
    "smat_gram_lists": (_i, [_i, _p, _p, _p, _p, _p, _i, _i, _i, _i64, _i64, _p]),
    "smat_query_lists": (_i, [_i, _p, _p, _p, _p, _p, _i, _i, _i, _i, _i64, _i64, _p]),
    "smat_cell_hash": (_i, [_i, _p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _i, _i, _i64, _i64, _p]),
    "smat_hash_pairs": (_i, [_p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _i, _p]),
    "smat_hash_pairs_backward": (_i, [_p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _i, _p]),
    "smat_zeta": (_i, [_p, _p, _i, _i, _i64, _p]),
    "smat_walsh": (_i, [_p, _p, _i, _i, _i64, _p]),
    "smat_incidence_complement": (_i, [_p, _p, _i, _i, _i, _i64, _p]),
    "smat_decode_step": (_i, [_i, _p, _p, _p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _i64,
                              _i64, _i64, _i64, _p]),
}

_lock = threading.Lock()
_lib = None


def load():
    """The loaded library (cached); raises :class:`HipUnavailable` if absent."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise HipUnavailable(
                f"{LIB_PATH} is not built; run `python -m smat_attention_amd._build` "
                f"(or __graft_entry__.build()) first")
        try:
            lib = ctypes.CDLL(LIB_PATH)
        except OSError as e:
            raise HipUnavailable(f"cannot load {LIB_PATH}: {e}") from e
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
        return lib


def exported_symbols():
    return list(SIGNATURES)


def call(name: str, *args) -> int:
    """Call entry point ``name``; raise :class:`HipKernelError` on a nonzero status."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != 0:
        msg = lib.smat_last_error().decode(errors="replace")
        raise HipKernelError(name, rc, msg)
    return rc


def query(name: str, *args) -> int:
    """Call a size query (returns a value, never fails)."""
    return int(getattr(load(), name)(*args))


def version() -> str:
    return load().smat_version().decode()


VARIANTS = {"scan": 0, "gram": 1, "query": 2, "incidence": 3, "incidence_plane": 4}


@contextlib.contextmanager
def general_kernel(name: str):
    """Within the block, run the general kernel that the specialised one named
    ``name`` (a key of :data:`VARIANTS`) replaced (``smat_set_variant``), then
    restore the previous choice.  A test hook: it switches every call made
    meanwhile, on every thread."""
    which = VARIANTS[name]
    lib = load()
    prev = lib.smat_set_variant(which, 1)
    if prev < 0:
        raise HipKernelError("smat_set_variant", prev, lib.smat_last_error().decode())
    try:
        yield
    finally:
        lib.smat_set_variant(which, prev)


STAGES = ("pool", "incidence", "query", "causal_scan")


@contextlib.contextmanager
def stage_events(events):
    """Within the block, every one-call forward (``smat_forward``,
    ``smat_forward_fused``) made on this thread binds ``events[i]`` (a
    ``torch.cuda.Event`` with timing, one per stage of :data:`STAGES`) to the
    end of stage i's last kernel, through the launch itself
    (``smat_set_stage_events``).  With an event recorded just before the call,
    consecutive events bracket each stage as the call ran it."""
    handles = []
    for e in events:
        if not e.cuda_event:
            e.record()                     # the handle exists once recorded
        handles.append(e.cuda_event)
    arr = (ctypes.c_void_p * len(handles))(*handles)
    call("smat_set_stage_events", arr, len(handles))
    try:
        yield
    finally:
        call("smat_set_stage_events", None, 0)


def stream_of(t: torch.Tensor) -> int:
    """hipStream_t of torch's current stream on ``t``'s device, as an integer."""
    return torch.cuda.current_stream(t.device).cuda_stream


def ptr(t) -> int:
    return 0 if t is None else t.data_ptr()
