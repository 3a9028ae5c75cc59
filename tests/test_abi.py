"""The C ABI library: it loads, exports every entry point include/smat_hip.h
declares, and rejects bad arguments before touching a GPU.  CPU only."""
import os
import re

import pytest

from smat_attention_amd.kernels import _lib
from smat_attention_amd.kernels._lib import HipKernelError

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "smat_hip.h")


def _declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^(?:int|int64_t|const char\*)\s+(smat_\w+)\(", text, re.M)))


def test_library_loads():
    lib = _lib.load()
    assert _lib.version().endswith("gfx950")
    assert lib.smat_last_error() == b""


def test_every_declared_symbol_is_exported_and_bound():
    lib = _lib.load()
    declared = _declared()
    assert declared, "no declarations parsed from the header"
    for name in declared:
        assert hasattr(lib, name), f"{name} declared but not exported"
    assert declared == sorted(_lib.SIGNATURES), "ctypes signature table differs from the header"


def test_header_argument_counts_match_bindings():
    text = open(HEADER).read()
    for name, (_, args) in _lib.SIGNATURES.items():
        m = re.search(rf"^(?:int|int64_t|const char\*)\s+{name}\((.*?)\);", text, re.M | re.S)
        assert m, name
        params = [p for p in m.group(1).split(",") if p.strip() and p.strip() != "void"]
        assert len(params) == len(args), f"{name}: header has {len(params)} args, binding {len(args)}"


def test_null_pointer_is_rejected_without_a_gpu():
    with pytest.raises(HipKernelError, match="null pointer"):
        _lib.call("smat_chunk_local", 0, None, None, None, None, None, 1, 128, 64, 65,
                  0, 64, 0, 64, 0, 65, 0, 65, 0, 65, None)


def test_unsupported_sizes_are_rejected():
    fake = 1 << 20      # never dereferenced: validation fails first
    with pytest.raises(HipKernelError) as e:
        _lib.call("smat_chunk_local", 0, fake, fake, fake, fake, fake, 1, 128, 256, 65,
                  0, 256, 0, 256, 0, 65, 0, 65, 0, 65, None)
    assert e.value.code == -2 and "r=256" in str(e.value)
    with pytest.raises(HipKernelError, match="unknown dtype"):
        _lib.call("smat_forward", 7, fake, fake, fake, fake, 0, None, 1, None, 0, fake, None,
                  None, 1, 256, 128, 0, 4, 4, 128, 16, 17, 0, 16, 0, 16, 0, 17, 0, 16, 0,
                  fake, 1 << 30, None)


def test_workspace_query_arithmetic():
    # C3 at T=131072, d=3, nb=8, r=128, p=129 (n=65536, N0=1681, B=1722)
    nb, T, n, N0, B, r, p, C = 8, 131072, 65536, 1681, 1722, 128, 129, 128
    ws = _lib.query("smat_forward_workspace_bytes", nb, T, n, N0, B, 0, C, r, p)
    rp4 = r * p * 4
    nc = T // C
    y_st = (p + 3) // 4 * 4          # the long-range term's rows are padded to 16 bytes
    # F and U rows are sized for the stride the line-group incidence takes: the
    # first odd multiple of 16 floats at or above r * p (16528 here)
    ld = (r * p + 15) // 16 * 16
    ld += 16 if (ld // 16) % 2 == 0 else 0
    assert ld == 16528
    expect_min = (nb * (N0 + B) * ld * 4 + nb * 2 * nc * rp4 + nb * (T - n) * y_st * 4
                  + nb * T * p * 4)
    assert expect_min <= ws <= expect_min + 16 * 256
    # d = 1 splits the single long progression: partial buffers appear
    assert _lib.query("smat_pool_workspace_bytes", 8, 0, 65536, 1, r, p) > 0
    assert _lib.query("smat_pool_workspace_bytes", 8, 0, 65536, 1681, r, p) == 0


def test_patch_swaps_the_kernel_table():
    """triton_bwd.patch()/unpatch() (triton_bwd.py:334-346): the differentiable
    wrappers replace chunk_local/pool/incidence in the kernel module and its
    reference-named alias, and are restored after."""
    from smat_attention_amd.kernels import hip_bwd, hip_fwd, triton_bwd, triton_fwd
    orig = (hip_fwd.chunk_local, hip_fwd.pool, hip_fwd.incidence)
    triton_bwd.patch()
    try:
        assert hip_bwd.patched()
        for mod in (hip_fwd, triton_fwd):
            assert mod.chunk_local is hip_bwd.chunk_local
            assert mod.pool is hip_bwd.pool
            assert mod.incidence is hip_bwd.incidence
        triton_bwd.patch()                     # idempotent
    finally:
        triton_bwd.unpatch()
    assert not hip_bwd.patched()
    assert (hip_fwd.chunk_local, hip_fwd.pool, hip_fwd.incidence) == orig
    assert (triton_fwd.chunk_local, triton_fwd.pool, triton_fwd.incidence) == orig
