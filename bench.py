#!/usr/bin/env python3
"""Benchmark of the SMat forward schedule on one MI355X.

Workload (the long-prefill configuration the metric is quoted on): B=1, H=8
(nb = 8 sequences x heads), head_dim 128 (feature rank r = 128, p = 129),
T = 131072, d = 3 geometric mask, chunk 128, bf16 inputs with fp32
accumulation and fp32 output; q, k, v ~ N(0, 1) drawn on the CPU from seed 0,
k scaled by 1/sqrt(128); features Phi = elu(q W^T) + 1, Psi = elu(k W^T) + 1,
Vb = [v, 1] computed before the timed region (the reference times prefill
without featurisation too).

A step is one full forward (pool -> incidence -> query -> causal scan ->
normalise) over the resident inputs.  W untimed steps, then K timed steps
between two device synchronisations.  Printed: one JSON line with the
throughput (tokens/s = B*T / step time), the roofline of the dominant kernel
(timed live with events on the stream the kernels run on), the CPU baseline
(the oracle's restatement of the reference's torch path, on a bounded
sample, timed on this host), the cached-decode rate and, outside the step,
the time of one content-hashed training step (forward and backward, B=8,
H=12, head_dim 64, T=4096, bf16, d = 2 and 3), the long prefill at every
T in {32768, 131072, 524288} with d = 3 and the d = 1 control, and cached
decode over 4096 steps after a 65536-token context (B=16, H=8).

    python bench.py [--steps K] [--warmup W] [--T 131072] [--no-cpu] [--no-decode]
                    [--no-train] [--no-rows]
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, GB/s
BF16_PEAK_TFLOPS = 2500.0      # MI355X dense bf16 MFMA, TFLOP/s
VALU_F32_ADD_PEAK_T = 39.32    # fp32 vector adds, 10^12/s: 1024 SIMDs x 16 lanes x 2.4 GHz

# HBM bytes per launch of a stage on a workload, measured with two rocprofv3
# counter passes (FETCH_SIZE, WRITE_SIZE) of `bench.py --copy-probe` and scaled by
# what the counters read for a 1 GiB device copy (x2.0 and x1.0); the passes are
# recorded under profiles/.  Keyed by (stage, T, d, heads, head_dim); each entry
# holds the sha256 prefix of the kernel source it was measured on, and is reported
# only while that source is unchanged.
MEASURED_TRAFFIC = {
    ("incidence", 131072, 3, 8, 128): ("csrc/incidence.hip", "986fa7556bdc4b06", 1_825_573_593),
    ("incidence", 524288, 3, 8, 128): ("csrc/incidence.hip", "986fa7556bdc4b06", 5_021_811_190),
}


def measured_traffic(stage, T, d, nb, hd):
    import hashlib
    ent = MEASURED_TRAFFIC.get((stage, T, d, nb, hd))
    if ent is None:
        return None
    src, sha, nbytes = ent
    path = os.path.join(ROOT, "smat_attention_amd", src)
    try:
        with open(path, "rb") as f:
            cur = hashlib.sha256(f.read()).hexdigest()[:16]
    except OSError:
        return None
    return nbytes if cur == sha else None

METRIC = "SMat prefill tokens/s at T=131072 bf16 d=3; % of MFMA peak; decode GB/s"


def parse():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--T", type=int, default=131072)
    ap.add_argument("--d", type=int, default=3)
    ap.add_argument("--heads", type=int, default=8)
    ap.add_argument("--head-dim", type=int, default=128)
    ap.add_argument("--kernel-reps", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-heads", type=int, default=2,
                    help="heads in the CPU baseline sample (of --heads)")
    ap.add_argument("--cpu-threads", type=int, default=16)
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--no-train", action="store_true", help="skip the training-step timing")
    ap.add_argument("--train-only", action="store_true",
                    help="time the training steps alone (for profiling): no prefill, decode, "
                         "CPU baseline or JSON line")
    ap.add_argument("--qkv-only", action="store_true",
                    help="time the path from q, k, v alone at --T / --d (for profiling): "
                         "featurise + smat_attention, then smat_attention_fused, "
                         "--kernel-reps calls each; no JSON line")
    ap.add_argument("--decode-steps", type=int, default=4096)
    ap.add_argument("--no-rows", action="store_true",
                    help="skip the per-T / d = 1 prefill rows")
    ap.add_argument("--row-steps", type=int, default=10)
    ap.add_argument("--clock-warmup", type=float, default=1.0,
                    help="seconds of untimed forward calls before the warm-up steps")
    ap.add_argument("--verbose", action="store_true")
    ap.add_argument("--copy-probe", action="store_true",
                    help="first copy a 1 GiB fp32 buffer 3 times: the known-size kernel "
                         "that scales FETCH_SIZE / WRITE_SIZE counters to bytes")
    return ap.parse_args()


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def make_inputs(nb, T, hd, dtype, seed=0):
    """Seeded CPU draw, featurised on the CPU in fp32, cast, then moved."""
    import torch
    from smat_attention_amd.attention import make_phi
    gen = torch.Generator(device="cpu").manual_seed(seed)
    Q = torch.randn(nb, T, hd, generator=gen)
    K = torch.randn(nb, T, hd, generator=gen) * hd ** -0.5
    V = torch.randn(nb, T, hd, generator=gen)
    W = make_phi(hd, hd, dtype=torch.float32, seed=0).W
    Phi = (torch.nn.functional.elu(Q @ W.T) + 1).to(dtype)
    Psi = (torch.nn.functional.elu(K @ W.T) + 1).to(dtype)
    Vb = torch.cat([V, torch.ones(nb, T, 1)], dim=-1).to(dtype)
    return Phi, Psi, Vb


def to_gpu_padded(Phi, Psi, Vb, dev):
    """Move to the device; Vb rows padded to a 16-byte multiple (same values)."""
    import torch
    p = Vb.shape[-1]
    pad = -(-p // 8) * 8
    buf = torch.zeros(*Vb.shape[:-1], pad, device=dev, dtype=Vb.dtype)
    buf[..., :p] = Vb.to(dev)
    return Phi.to(dev), Psi.to(dev), buf[..., :p]


def gpu_inputs(nb, T, hd, seed):
    """Seeded draw on the GPU, featurised by the HIP feature map in bf16:
    q, k, v ~ N(0, 1), k scaled by 1/sqrt(hd); Vb rows padded to 16 bytes."""
    import torch
    from smat_attention_amd import attention as A
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(seed)
    bf = torch.bfloat16
    Q = torch.randn(nb, T, hd, device=dev, generator=g).to(bf)
    K = (torch.randn(nb, T, hd, device=dev, generator=g) * hd ** -0.5).to(bf)
    V = torch.randn(nb, T, hd, device=dev, generator=g).to(bf)
    return A.featurise(Q, K, V, A.make_phi(hd, hd, device=dev, dtype=bf, seed=0))


def time_forward(spec, Phi, Psi, Vb, steps, warmup):
    """ms per forward (one library call, inputs resident), host clock between
    two device synchronisations."""
    import torch
    from smat_attention_amd import attention as A
    nb, T, r = Phi.shape
    ws = torch.empty(A._hip.forward_workspace_bytes(nb, T, spec.n, spec.N0, spec.B, spec.n_P,
                                                    128, r, Vb.shape[-1]) + 256,
                     device=Phi.device, dtype=torch.uint8)
    for _ in range(warmup):
        A.smat_attention(Phi, Psi, Vb, spec, workspace=ws)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        out = A.smat_attention(Phi, Psi, Vb, spec, workspace=ws)
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) / steps * 1e3
    assert torch.isfinite(out).all()
    return ms


def prefill_rows(args):
    """The long prefill at T in {32768, 131072, 524288}, d = 3 and the d = 1
    control (B=1, H=8, head_dim 128, bf16): ms, tokens/s, the fraction of the
    dense-bf16 MFMA peak on useful FLOPs, and the fraction of the schedule's
    roofline max(t_MFMA, t_HBM) on its compulsory bytes."""
    import torch
    from smat_attention_amd import attention as A
    from smat_attention_amd.mask import build_mask, estimate_cost
    nb, hd = args.heads, args.head_dim
    rows = {}
    for T in (32768, 131072, 524288):
        Phi, Psi, Vb = gpu_inputs(nb, T, hd, seed=T)
        for d in (3, 1):
            spec = A.to_device(build_mask(T, d, chunk=128), Phi.device)
            ms = time_forward(spec, Phi, Psi, Vb, args.row_steps, 5)
            est = estimate_cost(T, d, hd, hd, chunk=128)
            flops = nb * est["mfma_flops"]
            cbytes = nb * (est["inputs_bf16"] + est["output_fp32"])
            t_roof = max(flops / (BF16_PEAK_TFLOPS * 1e12), cbytes / (HBM_PEAK_GBS * 1e9))
            rows[f"T{T}_d{d}"] = {
                "ms": round(ms, 4), "tokens_per_s": round(T / (ms * 1e-3), 1),
                "mfma_frac_of_bf16_peak": round(flops / (ms * 1e-3) / (BF16_PEAK_TFLOPS * 1e12), 4),
                "schedule_roofline_frac": round(t_roof / (ms * 1e-3), 4),
                "q": spec.q, "B_types": spec.B, "nnz_C": spec.I_prof}
            log(f"[bench] prefill T={T} d={d}: {ms:.3f} ms, {T / ms / 1e3:.2f} M tok/s")
        del Phi, Psi, Vb
        torch.cuda.empty_cache()
    return rows


def fused_rows(args):
    """The long prefill from q, k, v, featurisation included (B=1, H=8,
    head_dim 128, bf16 q, k, v ~ N(0, 1), k scaled 1/sqrt(128), elu+1 map, no
    gates), at T in {32768, 131072, 524288}, d = 3 and 1: the reference's two
    passes (featurise, then the schedule; attention.py:82-106, :391-455) as
    featurise + smat_attention, against smat_attention_fused, whose kernels
    form Phi, Psi and [V, 1] in LDS.  ms per call (host clock between device
    synchronisations, inputs resident) and tokens/s of the fused call."""
    import torch
    from smat_attention_amd import attention as A
    from smat_attention_amd.kernels import _lib
    from smat_attention_amd.mask import build_mask
    nb, hd, steps = args.heads, args.head_dim, args.row_steps
    dev = torch.device("cuda:0")
    bf = torch.bfloat16
    phi = A.make_phi(hd, hd, device=dev, dtype=bf, seed=0)
    rows = {}

    def timed(fn):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            out = fn()
        torch.cuda.synchronize()
        assert torch.isfinite(out).all()
        return (time.perf_counter() - t0) / steps * 1e3

    for T in (32768, 131072, 524288):
        g = torch.Generator(device=dev).manual_seed(T + 7)
        Q = torch.randn(nb, T, hd, device=dev, generator=g).to(bf)
        K = (torch.randn(nb, T, hd, device=dev, generator=g) * hd ** -0.5).to(bf)
        V = torch.randn(nb, T, hd, device=dev, generator=g).to(bf)
        for d in (3, 1):
            spec = A.to_device(build_mask(T, d, chunk=128), dev)
            ws = torch.empty(_lib.query("smat_forward_fused_workspace_bytes", nb, T, spec.n,
                                        spec.N0, spec.B, spec.n_P, 128) + 256,
                             device=dev, dtype=torch.uint8)
            ms_u = timed(lambda: A.smat_attention(*A.featurise(Q, K, V, phi), spec))
            ms_f = timed(lambda: A.smat_attention_fused(Q, K, V, phi, spec, workspace=ws))
            rows[f"T{T}_d{d}"] = {"featurise_then_forward_ms": round(ms_u, 4),
                                  "fused_ms": round(ms_f, 4),
                                  "fused_kernels": A._fused_ok(Q, K, V, phi, spec, 128, None),
                                  "fused_tokens_per_s": round(T / (ms_f * 1e-3), 1),
                                  "speedup": round(ms_u / ms_f, 3)}
            log(f"[bench] q,k,v prefill T={T} d={d}: featurise + forward {ms_u:.3f} ms, "
                f"fused {ms_f:.3f} ms")
            del ws
        del Q, K, V
        torch.cuda.empty_cache()
    return rows


def qkv_bench(args):
    """The path from q, k, v at one (T, d): featurise + smat_attention, then
    smat_attention_fused, ``--kernel-reps`` calls each after 3 warm-up calls,
    bracketed by device synchronisations (inputs as in :func:`fused_rows`)."""
    import torch
    from smat_attention_amd import attention as A
    from smat_attention_amd.mask import build_mask
    nb, hd, T, reps = args.heads, args.head_dim, args.T, args.kernel_reps
    dev = torch.device("cuda:0")
    bf = torch.bfloat16
    g = torch.Generator(device=dev).manual_seed(T + 7)
    Q = torch.randn(nb, T, hd, device=dev, generator=g).to(bf)
    K = (torch.randn(nb, T, hd, device=dev, generator=g) * hd ** -0.5).to(bf)
    V = torch.randn(nb, T, hd, device=dev, generator=g).to(bf)
    phi = A.make_phi(hd, hd, device=dev, dtype=bf, seed=0)
    spec = A.to_device(build_mask(T, args.d, chunk=128), dev)
    for name, fn in (("featurise + smat_attention",
                      lambda: A.smat_attention(*A.featurise(Q, K, V, phi), spec)),
                     ("smat_attention_fused", lambda: A.smat_attention_fused(Q, K, V, phi, spec))):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(reps):
            fn()
        torch.cuda.synchronize()
        log(f"[bench] q,k,v T={T} d={args.d} {name}: "
            f"{(time.perf_counter() - t0) / reps * 1e3:.3f} ms")


class Events:
    """Per-kernel durations with events recorded on the stream the kernels use."""

    def __init__(self, torch):
        self.torch = torch

    def time(self, fn, reps):
        torch = self.torch
        fn()
        torch.cuda.synchronize()
        s = torch.cuda.current_stream()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(s)
        for _ in range(reps):
            fn()
        e1.record(s)
        e1.synchronize()
        return e0.elapsed_time(e1) / reps * 1e3      # microseconds per launch


def kernel_table(spec, Phi, Psi, us):
    """Algorithmic traffic/work of each stage of the one-call forward, priced
    at ``us``, the stage durations measured in the timed steps: each stage's
    last kernel launch binds an event to its end (smat_set_stage_events) --
    the pool, the incidence, the type-major query and the causal pass (the
    chunk-group Gram prepass, the group scan and the scan kernel that also adds
    Y, normalises and writes the output) -- so a stage is the time from the
    previous stage's end to its own (its kernels and the dispatch gap before
    them)."""
    nb, T, r = Phi.shape
    p = r + 1
    n, C, N0, B, T_R = spec.n, 128, spec.N0, spec.B, spec.T_R
    eb = Phi.element_size()
    rp4 = r * p * 4
    # algorithmic bytes: each operand read once and each result written once
    rows = {
        "pool": dict(us=us["pool"], bytes=nb * ((n - spec.n_P) * (r + p) * eb + N0 * rp4),
                     flops=2 * nb * (n - spec.n_P) * r * p),
        "incidence": dict(us=us["incidence"], bytes=nb * (N0 + B) * rp4,
                          flops=nb * spec.I_prof * r * p),
        "query": dict(us=us["query"], bytes=nb * (B * rp4 + T_R * r * eb + T_R * p * 4),
                      flops=2 * nb * T_R * r * p),
        "causal_scan": dict(
            us=us["causal_scan"],
            bytes=nb * (T * (2 * r + p) * eb + T_R * p * 4 + T * (p - 1) * 4),
            flops=2 * nb * (T * (C + 1) / 2 * (r + p) + 2 * T * r * p)),
    }
    for v in rows.values():
        v["GBs"] = v["bytes"] / (v["us"] * 1e-6) / 1e9
        v["TFLOPs"] = v["flops"] / (v["us"] * 1e-6) / 1e12
    return rows


def featurise_bench(nb, T, hd, reps):
    """Time the feature map and value packing (attention.py:82-106: Phi, the
    gated Psi and [V, 1] in one launch) on bf16 q, k, v and gate h ~ U[0.5, 1.5),
    as the reference's bench draws them (bench_prefill.py:189-198); the
    reference reports this as featurise_ms, outside the prefill time."""
    import torch
    from smat_attention_amd import attention as A
    dev = torch.device("cuda:0")
    gen = torch.Generator(device="cpu").manual_seed(1)
    Q, K, V = (torch.randn(nb, T, hd, generator=gen).to(dev, torch.bfloat16) for _ in range(3))
    h = (torch.rand(nb, T, generator=gen) + 0.5).to(dev, torch.bfloat16)
    phi = A.make_phi(hd, hd, device=dev, dtype=torch.bfloat16, seed=0)
    us = Events(torch).time(lambda: A.featurise(Q, K, V, phi, h=h), reps)
    nbytes = nb * T * 2 * (3 * hd + 2 * hd + (hd + 1) + 1)
    del Q, K, V, h
    return {"us": round(us, 1), "GBs": round(nbytes / (us * 1e-6) / 1e9, 1), "bytes": nbytes,
            "config": f"nb={nb} T={T} d_qk=r=d_v={hd} bf16, elu+1 map, key gate"}


def train_step_bench(d, reps, B=8, H=12, hd=64, T=4096):
    """One training step of the content-hashed layer, forward and backward, on
    bf16 q, k, v ~ N(0, 1) (k scaled by 1/sqrt(hd)) and an fp32 hidden state
    the hash reads (d_model = H*hd), upstream gradient dO ~ N(0, 1): the
    feature map, the segmented causal scan plus the content-addressed
    long-range term on the recent rows, the single division and the cast to
    bf16 (model.py:296-300, 317), then backward from dO (``o.backward(dO)``:
    the gradient the next layer hands back) to q, k, v, the hidden state and
    the hash parameters, their gradients cleared first as zero_grad
    (set_to_none) does; and the same step with positional assignment
    (smat_attention, the cast to bf16, forward and backward)."""
    import torch
    from smat_attention_amd import attention as A
    from smat_attention_amd.assign import ContentAssign
    from smat_attention_amd.mask import build_mask
    dev = torch.device("cuda:0")
    spec = build_mask(T, d, chunk=128)
    n = spec.n
    gen = torch.Generator(device="cpu").manual_seed(2)
    bf = torch.bfloat16
    Q = torch.randn(B * H, T, hd, generator=gen).to(dev, bf).requires_grad_(True)
    K = (torch.randn(B * H, T, hd, generator=gen) / hd ** 0.5).to(dev, bf).requires_grad_(True)
    V = torch.randn(B * H, T, hd, generator=gen).to(dev, bf).requires_grad_(True)
    X = torch.randn(B, T, H * hd, generator=gen).to(dev).requires_grad_(True)
    dO = torch.randn(B * H, T, hd, generator=gen).to(dev, bf)
    torch.manual_seed(7)
    m = ContentAssign(H, H * hd, spec, mode="point").to(dev)
    phi = A.make_phi(hd, hd, device=dev, dtype=bf, seed=0)

    def step():
        for t in (Q, K, V, X):                              # zero_grad(set_to_none=True)
            t.grad = None
        m.zero_grad(set_to_none=True)
        Phi, Psi, Vb = A.featurise(Q, K, V, phi)
        Hs = A.segmented_causal_scan(Phi, Psi, Vb, n, 128)
        # cat + clamped division + the cast to the model dtype
        o = A.combine_normalise(Hs, m(X, Phi, Psi, Vb, n), n, out_dtype=bf)
        o.backward(dO)
    us = Events(torch).time(step, reps)
    res = {"ms": round(us / 1e3, 3), "tokens_per_s": round(B * T / (us * 1e-6), 1),
           "config": f"B={B} H={H} head_dim={hd} T={T} d={d} bf16, content-hashed point read, "
                     f"fwd+bwd"}
    # the positional schedule on the same tensors: smat_attention forward and backward
    spec_t = A.to_device(spec, dev)

    def step_pos():
        for t in (Q, K, V):
            t.grad = None
        Phi, Psi, Vb = A.featurise(Q, K, V, phi)
        o = A.smat_attention(Phi, Psi, Vb, spec_t).to(bf)
        o.backward(dO)
    us = Events(torch).time(step_pos, reps)
    res["positional_ms"] = round(us / 1e3, 3)
    return res


def useful_flops(spec, nb, T, r, p, C=128):
    """Mask-density-scaled MFMA work of the schedule: causal intra-chunk QK^T and
    AV, Phi Sin, chunk summaries, pooling, type-major query (2 flops per MAC)."""
    macs = (T * (C + 1) / 2 * (r + p) + T * r * p + T * r * p
            + (spec.n - spec.n_P) * r * p + spec.T_R * r * p)
    return 2.0 * nb * macs


def compulsory_bytes(nb, T, r, p, eb_in=2, eb_out=4):
    return nb * (T * (2 * r + p) * eb_in + T * (p - 1) * eb_out)


def host_cpu_info():
    """CPU model, logical CPUs and physical cores visible to this process."""
    aff = sorted(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else []
    model, cores, cur = "", set(), {}
    try:
        with open("/proc/cpuinfo") as f:
            for line in f.read().splitlines() + [""]:
                if not line.strip():
                    if cur and (not aff or int(cur.get("processor", -1)) in aff):
                        cores.add((cur.get("physical id", "0"), cur.get("core id",
                                                                     cur.get("processor"))))
                        model = model or cur.get("model name", "")
                    cur = {}
                    continue
                k, _, v = line.partition(":")
                cur[k.strip()] = v.strip()
    except OSError:
        pass
    return {"cpu_model": model, "host_cpus": os.cpu_count(),
            "logical_cpus_visible": len(aff) or os.cpu_count(),
            "physical_cores_visible": len(cores) or None}


def _median_time(fn, runs=3):
    fn()                                            # one warm-up
    ts = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return statistics.median(ts)


def cpu_baseline(args, spec, Phi, Psi, Vb):
    """The oracle's restatement of the reference's torch path, timed on this
    host on bounded samples of each workload (median of 3 runs after one
    warm-up, as the reference's harness times, analysis/bench_prefill.py:81-102):

    * the long prefill at T = 131072 and T = 32768 (the first 32768 tokens of
      the same draw), d = 3 and d = 1, on ``cpu_heads`` of the heads, scaled to
      all heads (heads are independent);
    * cached decode: 8 of the 128 sequences, U from the 34816-token landmark
      block and the state of the rest of the 65536-token context (not timed),
      then 64 steps timed, scaled to 128 sequences;
    * the CPU plumbing configuration in full (nb = 4, T = 1024, d = 2, fp32).
    """
    import torch
    import oracle.schedule as O
    from smat_attention_amd.mask import build_mask
    info = host_cpu_info()
    threads = max(1, min(args.cpu_threads, info["physical_cores_visible"]
                         or info["logical_cpus_visible"] or 1))
    torch.set_num_threads(threads)
    nb, h = Phi.shape[0], args.cpu_heads
    rows = {}
    for T in dict.fromkeys((args.T, 32768)):
        P, S, W = (x[:h, :T].contiguous() for x in (Phi, Psi, Vb))
        for d in (3, 1):
            sp = spec if (T, d) == (args.T, args.d) else build_mask(T, d, chunk=128)
            t = _median_time(lambda: O.smat_attention(P, S, W, sp))
            t_all = t * nb / h
            rows[f"T{T}_d{d}"] = {"tokens_per_s": round(T / t_all, 1),
                                  "s_per_sample": round(t, 3)}
            log(f"[bench] cpu T={T} d={d}: {t:.3f} s for {h} heads")
    # decode: 8 sequences, 64 steps
    ns, hd = 8, args.head_dim
    dspec = build_mask(65536 + 4096, 3, chunk=128)
    n = dspec.n
    g = torch.Generator().manual_seed(3)
    feat = lambda *sh: (torch.nn.functional.elu(torch.randn(*sh, generator=g)) + 1
                        ).to(torch.bfloat16)
    vb = lambda *sh: torch.cat([torch.randn(*sh, hd, generator=g), torch.ones(*sh, 1)],
                               -1).to(torch.bfloat16)
    dec = O.SmatDecoder(feat(ns, n, hd), vb(ns, n), dspec)
    Pr, Vr = feat(ns, 65536 - n, hd), vb(ns, 65536 - n)
    dec.S = Pr.float().transpose(-1, -2) @ Vr.float()
    dec.i = 65536 - n
    steps = 64
    ph, ps, vv = feat(steps, ns, hd), feat(steps, ns, hd), vb(steps, ns)

    def run_steps():
        for i in range(steps):
            dec.step(ph[i], ps[i], vv[i])
    t = _median_time(run_steps)
    rows["decode"] = {"us_per_step": round(t / steps * 1e6 * 128 / ns, 1),
                      "sample": f"{ns} of 128 sequences, {steps} steps, scaled x{128 // ns}"}
    log(f"[bench] cpu decode: {rows['decode']}")
    # CPU plumbing configuration in full
    sp1 = build_mask(1024, 2, chunk=128)
    Q1, K1, V1 = O.seeded_qkv(4, 1024, 64, 64, seed=0)
    P1, S1, W1 = O.featurise(Q1, K1, V1, O.make_phi(64, 64, seed=0))
    t = _median_time(lambda: O.smat_attention(P1, S1, W1, sp1))
    rows["plumbing_T1024_d2_fp32"] = {"ms": round(t * 1e3, 2),
                                      "tokens_per_s": round(4 * 1024 / t, 1)}
    main_row = rows[f"T{args.T}_d{args.d}"]
    return {"value": main_row["tokens_per_s"], "unit": "tokens/s", "cores": threads,
            "kind": "port",
            "sample": (f"{h} of {nb} heads at T={args.T}, d={args.d}, bf16 inputs (reference "
                       f"torch path restated, oracle/schedule.py); median of 3 after 1 "
                       f"warm-up = {main_row['s_per_sample']} s, scaled x{nb // h} to all heads"),
            **info, "threads": threads, "rows": rows}


def decode_bench(args):
    """Cached decode at B=16, H=8 (nb = 128), head_dim 128, d = 3: a 65536-token
    context, then ``decode_steps`` (4096) steps, bf16 q, k, v ~ N(0, 1) drawn on
    the GPU and featurised there.  The mask covers all 69632 tokens (q = 37,
    B = 1406, n = 34816).  U is built from the landmark block and the
    context's recent tokens enter the state in one advance(); every step has
    its own inputs.  The steps are captured once into a HIP graph and replayed
    (no host launch cost between steps); the same steps launched eagerly are
    timed on a second decoder."""
    import torch
    from smat_attention_amd import attention as A
    from smat_attention_amd.mask import build_mask
    dev = torch.device("cuda:0")
    nb, hd, T_pre = 128, 128, 65536
    T_total = T_pre + 4096
    steps = min(args.decode_steps, 4096)
    steps -= steps % 2           # an even count returns the state to its first buffer
    spec = A.to_device(build_mask(T_total, 3, chunk=128), dev)
    r, p, n = hd, hd + 1, spec.n
    Phi, Psi, Vb = gpu_inputs(nb, T_total, hd, seed=7)
    s = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    out = torch.empty(nb, p - 1, device=dev)

    def decoder():
        dec = A.SmatDecoder(Psi[:, :n], Vb[:, :n], spec)
        dec.advance(Psi[:, n:T_pre], Vb[:, n:T_pre])
        return dec

    dec = decoder()
    eager = min(steps, 512)
    for i in range(8):
        dec.step(Phi[:, T_pre + i], Psi[:, T_pre + i], Vb[:, T_pre + i], out=out)
    torch.cuda.synchronize()
    e0.record(s)
    for i in range(eager):
        dec.step(Phi[:, T_pre + i], Psi[:, T_pre + i], Vb[:, T_pre + i], out=out)
    e1.record(s)
    e1.synchronize()
    us_eager = e0.elapsed_time(e1) / eager * 1e3
    del dec
    dec = decoder()
    graph = torch.cuda.CUDAGraph()
    cap = torch.cuda.Stream()
    cap.wait_stream(s)
    with torch.cuda.stream(cap):
        with torch.cuda.graph(graph, stream=cap):
            for i in range(steps):
                dec.step(Phi[:, T_pre + i], Psi[:, T_pre + i], Vb[:, T_pre + i], out=out)
    s.wait_stream(cap)
    graph.replay()                  # the 4096 decode steps after the context
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    e0.record(s)
    graph.replay()                  # the same work again (state carries on), timed
    e1.record(s)
    e1.synchronize()
    us = e0.elapsed_time(e1) / steps * 1e3
    # per step and sequence: U[type] read, S read, S write (r*p fp32 each), plus io
    step_bytes = nb * (3 * r * p * 4 + (2 * r + p) * 2 + (p - 1) * 4)
    return {"us_per_step": round(us, 2), "GBs": round(step_bytes / (us * 1e-6) / 1e9, 1),
            "frac_hbm": round(step_bytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
            "us_per_step_eager": round(us_eager, 2),
            "config": f"nb=128 (B=16,H=8), r=128, p=129, d=3, context {T_pre} then {steps} "
                      f"steps, B_types={spec.B}, replayed from one HIP graph",
            "bytes_per_step": step_bytes, "U_cache_GB": round(dec.U.numel() * 4 / 1e9, 2)}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}): this build has no "
              f"multi-GPU path; heads would shard across GPUs with no communication.",
              file=sys.stderr)
        sys.exit(2)
    import torch
    from smat_attention_amd import attention as A
    from smat_attention_amd.mask import build_mask

    if not A.have_hip():
        raise SystemExit("the HIP library or the GPU is missing; build with "
                         "`python -m smat_attention_amd._build` and run on the MI355X")
    dev = torch.device("cuda:0")
    if args.copy_probe:
        x = torch.ones(1 << 28, device=dev)
        y = torch.empty_like(x)
        for _ in range(3):
            y.copy_(x)
        torch.cuda.synchronize()
        del x, y
        log("[bench] copy probe: 3 x 1 GiB device copies")
    if args.train_only:
        for d in (2, 3):
            log(f"[bench] train step d={d}: {train_step_bench(d, max(3, args.kernel_reps // 2))}")
        return
    if args.qkv_only:
        qkv_bench(args)
        return
    nb, T, hd = args.heads, args.T, args.head_dim
    r, p = hd, hd + 1
    spec = build_mask(T, args.d, chunk=128)
    log(f"[bench] {spec.summary()}; nb={nb} r={r} p={p}")
    Phi_c, Psi_c, Vb_c = make_inputs(nb, T, hd, torch.bfloat16)
    Phi, Psi, Vb = to_gpu_padded(Phi_c, Psi_c, Vb_c, dev)
    A.to_device(spec, dev)
    ws = torch.empty(A._hip.forward_workspace_bytes(nb, T, spec.n, spec.N0, spec.B, spec.n_P,
                                                    128, r, p) + 256,
                     device=dev, dtype=torch.uint8)
    out = None
    # bring the GPU's clocks and power to the steady state of back-to-back
    # forwards before anything is timed: about a second of them (untimed, in
    # bursts of 16 between synchronisations), then the W warm-up steps.  A
    # forward followed by an idle host gap runs at another power state, and the
    # first back-to-back forwards after it run up to 20 % slower for ~10 steps.
    t_warm = time.perf_counter()
    while time.perf_counter() - t_warm < args.clock_warmup:
        for _ in range(16):
            A.smat_attention(Phi, Psi, Vb, spec, workspace=ws)
        torch.cuda.synchronize()
    for _ in range(args.warmup):
        out = A.smat_attention(Phi, Psi, Vb, spec, workspace=ws)
    torch.cuda.synchronize()
    log(f"[bench] warmup done ({args.clock_warmup:.1f} s of clock warm-up, {args.warmup} steps)")
    # every timed step binds one event per stage to the end of that stage's
    # last kernel (smat_set_stage_events); step k's pool runs from step k-1's
    # last event (the first from one recorded before the loop)
    from smat_attention_amd.kernels import _lib
    stages = _lib.STAGES
    cur = torch.cuda.current_stream()
    first = torch.cuda.Event(enable_timing=True)
    marks = [[torch.cuda.Event(enable_timing=True) for _ in stages] for _ in range(args.steps)]
    for e in [first] + [e for m in marks for e in m]:
        e.record(cur)                            # create the handles before timing
    torch.cuda.synchronize()
    first.record(cur)
    t0 = time.perf_counter()
    for m in marks:
        with _lib.stage_events(m):
            out = A.smat_attention(Phi, Psi, Vb, spec, workspace=ws)
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    ms = dt / args.steps * 1e3
    tokens_per_s = T / (ms * 1e-3)                # B*T tokens per step, B = 1
    log(f"[bench] {args.steps} steps: {ms:.3f} ms/step, {tokens_per_s / 1e6:.2f} M tokens/s")
    assert torch.isfinite(out).all()
    ends = [first] + [m[-1] for m in marks]
    stage_us = {k: statistics.fmean((marks[j][i - 1] if i else ends[j]).elapsed_time(marks[j][i])
                                    for j in range(args.steps)) * 1e3
                for i, k in enumerate(stages)}
    rows = kernel_table(spec, Phi, Psi, stage_us)
    for k, v in rows.items():
        log(f"[bench] {k:13s} {v['us']:9.1f} us  {v['GBs']:7.0f} GB/s  {v['TFLOPs']:6.1f} TF/s")
    # the roofline is one kernel's: causal_scan is three launches (the prepass,
    # the segment scan and the streaming scan), so the longest one-launch stage
    dom = max(("pool", "incidence", "query"), key=lambda k: rows[k]["us"])
    drow = rows[dom]
    traffic = measured_traffic(dom, T, args.d, nb, hd)
    uf = useful_flops(spec, nb, T, r, p)
    cb = compulsory_bytes(nb, T, r, p)
    t_mfma = uf / (BF16_PEAK_TFLOPS * 1e12)
    t_hbm = cb / (HBM_PEAK_GBS * 1e9)
    result = {
        "metric": METRIC,
        "value": round(tokens_per_s, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) q,k,v; random-init feature map)",
        "config": {"workload": f"long prefill d={args.d}: B=1 H={nb} head_dim={hd} T={T} "
                               f"chunk=128 bf16 in / fp32 acc+out",
                   "T": T, "d": args.d, "nb": nb, "r": r, "p": p, "q": spec.q, "N0": spec.N0,
                   "B_types": spec.B, "nnz_C": spec.I_prof, "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "kernel": dom,
                     "achieved": round(drow["GBs"], 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(drow["GBs"] / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "traffic_source": ("rocprofv3 FETCH_SIZE / WRITE_SIZE passes of this "
                                        "workload (profiles/), scaled by a 1 GiB copy; "
                                        "reported only while the kernel source's sha256 "
                                        "matches the one measured, not measured in this run"),
                     "us_per_launch": round(drow["us"], 2),
                     "timing": "in the timed steps: from the end of the previous stage's "
                               "kernel to the end of this one, events bound by the launches "
                               "inside the one-call forward (smat_set_stage_events), mean "
                               "over the steps",
                     "algorithmic_bytes_per_launch": int(drow["bytes"])},
        "mfma": {"useful_flops": uf, "achieved_TFLOPs": round(uf / (ms * 1e-3) / 1e12, 2),
                 "frac_of_bf16_peak": round(uf / (ms * 1e-3) / (BF16_PEAK_TFLOPS * 1e12), 4),
                 "schedule_roofline_frac": round(max(t_mfma, t_hbm) / (ms * 1e-3), 4),
                 "compulsory_bytes": cb},
        "kernels_us": {k: round(v["us"], 1) for k, v in rows.items()},
        "stages_sum_ms": round(sum(v["us"] for v in rows.values()) / 1e3, 4),
    }
    if dom == "incidence":
        # priced against HBM, but limited on chip: fp32 vector adds and LDS reads
        result["roofline"]["limited_by"] = "VALU issue and LDS reads (rocprofv3 counters)"
        # the same launch against the vector ALUs' fp32 add rate: 256 CUs x 4 SIMDs
        # x 16 lanes per clock at 2.4 GHz (one wave64 add per SIMD per 4 clocks)
        adds = drow["flops"]
        result["roofline"]["valu"] = {
            "adds_per_launch": int(adds),
            "achieved_Tadd_s": round(adds / (drow["us"] * 1e-6) / 1e12, 2),
            "peak_Tadd_s": VALU_F32_ADD_PEAK_T,
            "frac": round(adds / (drow["us"] * 1e-6) / 1e12 / VALU_F32_ADD_PEAK_T, 4)}
    result["featurise"] = featurise_bench(nb, T, hd, args.kernel_reps)
    log(f"[bench] featurise {result['featurise']}")
    del ws, out, Phi, Psi, Vb
    torch.cuda.empty_cache()
    if not args.no_rows:
        result["prefill_rows"] = prefill_rows(args)
        result["prefill_qkv_rows"] = fused_rows(args)
    if not args.no_train:
        result["train_step"] = {f"d{d}": train_step_bench(d, max(3, args.kernel_reps // 2))
                                for d in (2, 3)}
        log(f"[bench] train step {result['train_step']}")
    torch.cuda.empty_cache()
    if not args.no_decode:
        result["decode"] = decode_bench(args)
        log(f"[bench] decode {result['decode']}")
    if not args.no_cpu:
        log("[bench] CPU baseline ...")
        result["cpu_baseline"] = cpu_baseline(args, spec, Phi_c, Psi_c, Vb_c)
        log(f"[bench] cpu {result['cpu_baseline']}")
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
