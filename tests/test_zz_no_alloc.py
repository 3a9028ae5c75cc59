"""smat_causal_scan_noalloc (the entry point that allocates nothing) against
smat_causal_scan (the one with a caller workspace), both called through the C
ABI on the same inputs: two calls in a row, the second on a smaller input, so
the second call reuses the scratch array the first one left full.

Tolerance: 1e-5 relative to the largest output (the fp32 bar).  When the
scratch array forces longer chunk groups than the workspace entry point uses,
the group summaries are summed in a different association, so the results may
differ by fp32 rounding; with the same grouping they are the same kernels on
the same data.
"""
import pytest
import torch

from smat_attention_amd.kernels import _lib
from smat_attention_amd.kernels._lib import DTYPE_CODE, HipKernelError

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _inputs(nb, T, hd, dt, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    Phi = torch.rand(nb, T, hd, device=DEV, generator=g).to(dt) + 0.05
    Psi = torch.rand(nb, T, hd, device=DEV, generator=g).to(dt) + 0.05
    p = hd + 1
    pad = -(-p // 8) * 8
    Vbuf = torch.ones(nb, T, pad, device=DEV, dtype=dt)
    Vbuf[..., :hd] = torch.randn(nb, T, hd, device=DEV, generator=g).to(dt)
    return Phi, Psi, Vbuf[..., :p]


def _args(Phi, Psi, Vb, Y, gate, out, n, C, write_H):
    nb, T, r = Phi.shape
    p = Vb.shape[-1]
    return (DTYPE_CODE[Phi.dtype], Phi.data_ptr(), Psi.data_ptr(), Vb.data_ptr(),
            Y.data_ptr() if Y is not None else None,
            gate.data_ptr() if gate is not None else None, out.data_ptr(),
            nb, T, n, C, r, p, Phi.stride(0), Phi.stride(1), Psi.stride(0), Psi.stride(1),
            Vb.stride(0), Vb.stride(1),
            Y.stride(0) if Y is not None else 0, Y.stride(1) if Y is not None else 0,
            out.stride(0), out.stride(1), gate.stride(0) if gate is not None else 0,
            int(write_H))


def _both(nb, T, n, hd, dt, write_H, seed):
    """Run both entry points on one input; return (workspace result, no-alloc result)."""
    print(f"[case] no-alloc causal scan nb={nb} T={T} n={n} hd={hd} {dt} write_H={write_H}",
          flush=True)
    Phi, Psi, Vb = _inputs(nb, T, hd, dt, seed)
    p, C = hd + 1, 128
    Y = gate = None
    if not write_H:
        g = torch.Generator(device=DEV).manual_seed(seed + 1)
        Y = torch.rand(nb, T - n, -(-p // 4) * 4, device=DEV, generator=g)[..., :p]
        gate = torch.rand(nb, T, device=DEV, generator=g) + 0.5
    width = p if write_H else p - 1
    stream = torch.cuda.current_stream(DEV).cuda_stream
    ref = torch.empty(nb, T, width, device=DEV)
    wsb = _lib.query("smat_causal_scan_workspace_bytes", nb, T, C, hd, p)
    ws = torch.empty(wsb + 256, device=DEV, dtype=torch.uint8)
    base = (ws.data_ptr() + 255) & ~255
    _lib.call("smat_causal_scan", *_args(Phi, Psi, Vb, Y, gate, ref, n, C, write_H),
              base, wsb, stream)
    got = torch.full((nb, T, width), float("nan"), device=DEV)
    _lib.call("smat_causal_scan_noalloc", *_args(Phi, Psi, Vb, Y, gate, got, n, C, write_H),
              stream)
    torch.cuda.synchronize()
    return ref, got, wsb


def _rel(a, b):
    return ((a.double() - b.double()).abs().max() / b.double().abs().max()).item()


def test_noalloc_matches_workspace_entry_point_twice():
    """First a long sequence batch whose default grouping needs more scratch than
    the array holds (nb = 8, T = 131072, head_dim 128, bf16: 136 MB of group
    states), then a smaller fp32 input on the same array."""
    cap = _lib.query("smat_causal_scan_noalloc_max_bytes")
    assert cap == 64 << 20
    ref, got, wsb = _both(8, 131072, 65536, 128, torch.bfloat16, False, seed=3)
    assert wsb > cap                                # the regrouped path
    e1 = _rel(got, ref)
    print(f"  rel diff {e1:.2e}", flush=True)
    assert torch.isfinite(got).all() and e1 < 1e-5
    del ref, got
    ref, got, wsb = _both(2, 4096, 2048, 64, torch.float32, True, seed=4)
    assert wsb <= cap                               # the workspace path's own grouping
    e2 = _rel(got, ref)
    print(f"  rel diff {e2:.2e}", flush=True)
    assert torch.isfinite(got).all() and e2 < 1e-5


def test_noalloc_refuses_what_does_not_fit():
    """255 sequences of 128 x 129 states exceed the array even with one group
    per segment (254 fit): a clear error before any launch."""
    fake = 1 << 20          # never dereferenced: the size check fails first
    with pytest.raises(HipKernelError, match="scratch array"):
        _lib.call("smat_causal_scan_noalloc", 0, fake, fake, fake, None, None, fake,
                  255, 4096, 2048, 128, 128, 129, 0, 128, 0, 128, 0, 136, 0, 0, 0, 128, 0,
                  0, None)
