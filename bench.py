"""Benchmark of the fine-tuning kernel hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--kernels rope,swiglu,...]
                    [--no-cpu-baseline] [--only-launches]

A step is one fwd+bwd pass of a kernel's drop-in autograd path over one batch
of synthetic input already resident in HBM.  The
HBM-bound legs (RoPE, SwiGLU, GeGLU, RMSNorm) time their steps sustained:
steps back to back, step i on input set i % K where the K sets exceed 1.2 GB
(several times the 256 MB Infinity Cache), so no input is cached when a step
reads it and each step's writes drain to HBM during the next one; one pair of
HIP events brackets all the steps, which the host queues behind a GPU delay
sized to its own enqueue time, so the device runs them without host gaps
(the host-inclusive `wall_ms_per_step` is reported beside).  Inputs a step
overwrites (the in-place
backwards) become that set's next inputs (finite values; the kernels' cost
does not depend on them).  These legs also report `cold`: each step alone
after a read of a 512 MB buffer (the reference's RoPE benchmark flushes a
256 MB buffer before every rep, kernels/rope/benchmarks/bench_v3.py:310,
371), whose writes can still sit in the Infinity Cache when its end event
fires.  The cross-entropy and MFMA-bound legs time each step cold and alone
(the reference's CE benchmark times a rep alone,
kernels/cross_entropy/benchmarks/bench_cross_entropy.py:197-210); the 2.1 GB
CE logits are restored into one buffer before each step, outside the timed
interval.

The launch loops behind `roofline` time one launch of the dominant kernel.
For the HBM-bound legs they are sustained: launches back to back over
rotating buffer sets whose footprint (> 1.2 GB) is several times the
Infinity Cache, so no input is cached and earlier launches' writes drain to
HBM during later ones (a cold launch after a read-only flush can instead
leave its writes in the Infinity Cache past its end event).  These legs also
report `copy_ceiling`: a plain device copy of the same byte count timed both
ways.  The MFMA-bound launch loops are cold (a 512 MB read before each).
Every kernel is timed; the headline `value` is the RoPE fwd+bwd
throughput on configs[1] (B=4, S=4096, 32/8 heads, D=128, bf16, bases 10000
and 500000 alternate by step), the others are reported under "kernels".

roofline.achieved = algorithmic bytes (or FLOPs) per launch of the kernel's
dominant device kernel / its average launch duration, measured with HIP
events on the stream the kernel is launched on.  roofline.traffic comes from
profiles/traffic.json (rocprofv3 FETCH_SIZE + WRITE_SIZE per dispatch, scaled
by the copy-kernel calibration) when present, else null.
cpu_baseline: the oracle (the reference's PyTorch path restated, oracle/) on
the host cores on a bounded sample of the same workload (about 10 s of CPU
work per kernel, median per call), scaled to the metric.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "kernel-pocs_amd"))

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
METRIC = "fwd+bwd GB/s (% of HBM peak) for SwiGLU/RoPE/CE; LoRA-MLP MFMA TFLOPS"


def _parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--kernels",
                    default="swiglu,rope,ce,lora_mlp,lora_qkv,flce,geglu,rmsnorm,lora_patch,lora_mlp_geglu,lora_patch_gemma")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--only-launches", action="store_true",
                    help="run only the dominant-kernel launch loop (for rocprofv3 counter runs)")
    return ap.parse_args()


# ---------------------------------------------------------------------------
# timing helpers
# ---------------------------------------------------------------------------
def _sync():
    import torch

    torch.cuda.synchronize()


def time_steps(step_fn, steps, warmup):
    """Warm timing: warmup + steps back to back; returns (event ms per step
    over one timed bracket, wall ms per step)."""
    import torch

    for i in range(warmup):
        step_fn(i)
    _sync()
    t0 = time.perf_counter()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(warmup, warmup + steps):
        step_fn(i)
    end.record()
    _sync()
    wall = (time.perf_counter() - t0) * 1e3 / steps
    return start.elapsed_time(end) / steps, wall


SCRUB_BYTES = 512 << 20  # twice the 256 MB Infinity Cache
_SCRUB = []


def scrub():
    """Queues a read of a 512 MB buffer: afterwards neither the L2s nor the
    Infinity Cache hold any of the previous working set."""
    import torch

    if not _SCRUB:
        _SCRUB.append(torch.zeros(SCRUB_BYTES // 4, device="cuda"))
    _SCRUB[0].sum()


def time_steps_cold(step_fn, steps, warmup, restore_fn=None):
    """Per-step cold timing, the way the reference's benchmarks time one rep
    (a cache flush before each rep, HIP events around the rep alone:
    kernels/rope/benchmarks/bench_v3.py:310, 371;
    kernels/cross_entropy/benchmarks/bench_cross_entropy.py:197-210).
    restore_fn(i), if given, first rewrites the input buffer the step
    overwrites (the same buffer every step, as a training step gets the same
    block back from the caching allocator).  The 512 MB read then evicts
    everything the step will touch.  The host queues restore, read and step
    without waiting, so the events time the step's device work (the
    reference synchronizes before each rep, which also puts the host's
    launch latency inside its interval).  Returns (mean event ms over the K
    steps, wall ms per step including restores and reads)."""
    import torch

    for i in range(warmup):
        if restore_fn is not None:
            restore_fn(i)
        step_fn(i)
    _sync()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    t0 = time.perf_counter()
    for j, (a, b) in enumerate(evs):
        if restore_fn is not None:
            restore_fn(warmup + j)
        scrub()
        a.record()
        step_fn(warmup + j)
        b.record()
    _sync()
    wall = (time.perf_counter() - t0) * 1e3 / steps
    return statistics.mean(a.elapsed_time(b) for a, b in evs), wall


def time_launches(launch_fn, n, warmup=3):
    """Average duration (ms) of one device launch, cold (a 512 MB read before
    each, untimed), from events recorded on torch's current stream (the
    stream every forge_* call launches on)."""
    import torch

    for i in range(warmup):
        launch_fn(i)
    _sync()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n)]
    for i, (a, b) in enumerate(evs):
        scrub()
        a.record()
        launch_fn(i)
        b.record()
    _sync()
    return statistics.mean(a.elapsed_time(b) for a, b in evs)


SUSTAINED_FOOTPRINT = 1200 * 10 ** 6  # bytes of rotating buffers: > 4x the Infinity Cache
SUSTAINED_LABEL = "sustained: launches back to back over rotating buffer sets of > 1.2 GB"


def n_sets(set_bytes):
    """Buffer sets a sustained launch loop rotates over: at least two, and
    enough that their footprint exceeds SUSTAINED_FOOTPRINT."""
    return max(2, -(-SUSTAINED_FOOTPRINT // max(1, set_bytes)))


def time_sustained(launch_fn, n, warmup=4):
    """Average duration (ms) of one launch at steady state: launches run back
    to back, launch i on buffer set i % K (launch_fn picks it), where the K
    sets (> 1.2 GB) are several times the 256 MB Infinity Cache, so no input
    is cached when a launch reads it and the writes of earlier launches drain
    to HBM during later ones.  One pair of HIP events on torch's current
    stream (the stream every forge_* call launches on) brackets the n
    launches, which run with no gap between them; the mean is total / n.
    (An event pair around each launch would add the ~3-6 us that each event
    puts between two kernels.)"""
    import torch

    for i in range(warmup):
        launch_fn(i)
    _sync()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for i in range(n):
        launch_fn(warmup + i)
    b.record()
    _sync()
    return a.elapsed_time(b) / n


def copy_ceiling(args, nbytes, n=20):
    """Plain device copies moving nbytes in all (between buffers of nbytes / 2),
    timed both ways a kernel of the same byte count is: cold (after a 512 MB
    read, as the steps) and sustained (rotating sets, as the roofline
    launches).  Two copies: forge_copy (16-byte nontemporal loads and stores)
    and torch's elementwise kernel (y = x * 1 in bf16); the ceiling is the
    faster of the two.  A cold launch's writes can land in the Infinity Cache
    and drain after its end event; the copies are timed the same way, so the
    rates compare."""
    import torch
    from forge_hip import _lib as L

    if args.only_launches:
        return None
    half = nbytes // 2 // 16 * 16
    k = n_sets(2 * half)
    srcs = [torch.ones(half // 2, dtype=torch.bfloat16, device="cuda") for _ in range(k)]
    dsts = [torch.empty_like(s) for s in srcs]
    st = L.stream_of(srcs[0])
    fns = {
        "forge_copy": lambda i: L.forge_copy(dsts[i % k].data_ptr(), srcs[i % k].data_ptr(), half, st),
        "torch_mul": lambda i: torch.mul(srcs[i % k], 1, out=dsts[i % k]),
    }
    res = {"unit": "GB/s", "bytes": 2 * half}
    for name, fn in fns.items():
        cold_ms = time_launches(lambda i: fn(0), n)
        sus_ms = time_sustained(fn, n)
        res[name] = {"cold": rate(2 * half, cold_ms, 1e9), "sustained": rate(2 * half, sus_ms, 1e9)}
    res["cold"] = max(v["cold"] for v in (res["forge_copy"], res["torch_mul"]))
    res["sustained"] = max(v["sustained"] for v in (res["forge_copy"], res["torch_mul"]))
    del srcs, dsts
    return res


def run_steps(args, step_fn, restore=None):
    """Cold per-step timing (time_steps_cold); (None, None) with
    --only-launches."""
    if args.only_launches:
        return None, None
    return time_steps_cold(step_fn, args.steps, args.warmup, restore)


STEP_SUSTAINED_LABEL = ("sustained steps: back to back, step i on input set i % K, the K sets over 1.2 GB "
                        "(nothing cached; each step's writes drain during the next)")


def sustained_steps(args, step_fn):
    """The HBM legs' step figure: steps back to back, step_fn(i) on its
    input set i % K (the K sets exceed 1.2 GB, several times the 256 MB
    Infinity Cache, so no input is cached and the writes of each step drain
    to HBM during the next), one event pair around all of them.  The host
    queues the steps behind a GPU delay (torch.cuda._sleep) sized to its own
    measured enqueue time, so the device runs them without host gaps, as in
    a training loop whose host runs ahead; wall ms per step (host-inclusive,
    steps enqueued one after another) is reported beside.  Returns (ms per
    step, wall ms per step), or (None, None) with --only-launches."""
    import torch

    if args.only_launches:
        return None, None
    for i in range(args.warmup):
        step_fn(i)
    _sync()
    t0 = time.perf_counter()
    for i in range(args.warmup, 2 * args.warmup):
        step_fn(i)
    _sync()
    wall = (time.perf_counter() - t0) * 1e3 / args.warmup
    base = 2 * args.warmup
    # GPU delay covering the enqueue of all steps (1.5x the measured host
    # time per step, at most 200 ms; the sleep counts shader clocks)
    delay_s = min(0.2, 1.5 * wall * 1e-3 * args.steps + 1e-3)
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    torch.cuda._sleep(int(delay_s * 2.5e9))
    start.record()
    for j in range(args.steps):
        step_fn(base + j)
    end.record()
    _sync()
    return start.elapsed_time(end) / args.steps, wall


def cold_figure(args, step_fn, bytes_step, restore=None):
    """Each step alone after a 512 MB read (labelled, not the claim): its
    writes can still sit in the Infinity Cache when its end event fires."""
    if args.only_launches:
        return None
    ms, _ = time_steps_cold(step_fn, args.steps, args.warmup, restore)
    return {"value": rate(bytes_step, ms, 1e9), "unit": "GB/s", "ms_per_step": rnd(ms, 5),
            "timing": "cold: each step alone after a 512 MB read"}


def rate(amount, ms, scale):
    """amount per second / scale, or None when the step loop was skipped."""
    return None if ms is None else round(amount / (ms * 1e-3) / scale, 1)


def rnd(x, n):
    return None if x is None else round(x, n)


CPU_BUDGET_S = 10.0


def cpu_time(fn, budget_s=CPU_BUDGET_S, min_reps=3):
    """Median seconds per call of fn on the host: one untimed call, then
    repeated calls until about budget_s of CPU work (at least min_reps).
    Returns (median, reps)."""
    fn()
    ts = []
    t_start = time.perf_counter()
    while len(ts) < min_reps or time.perf_counter() - t_start < budget_s:
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return statistics.median(ts), len(ts)


def _traffic(name):
    p = ROOT / "profiles" / "traffic.json"
    if not p.exists():
        return None
    try:
        return json.loads(p.read_text()).get(name, {}).get("bytes_per_launch")
    except Exception:
        return None


# ---------------------------------------------------------------------------
# kernels
# ---------------------------------------------------------------------------
def bench_swiglu(args):
    """fp32 gate/up/dout [2048, 11008], out = silu(gate)*up."""
    import torch
    from forge_hip import _lib as L
    from kernels.swiglu import swiglu

    R, C = 2048, 11008
    n = R * C
    g = torch.Generator(device="cuda").manual_seed(0)
    gate0 = torch.randn(R, C, device="cuda", generator=g)
    up0 = torch.randn(R, C, device="cuda", generator=g)
    dout = torch.randn(R, C, device="cuda", generator=g)
    bytes_step = 8 * n * 4  # fwd 3 tensors + bwd 5 tensors, fp32
    # input sets (gate, up, dout) for the steps; the backward writes the
    # gradients over gate / up (the reference's in-place contract), which the
    # set's next step then takes as its input (finite values; the kernels'
    # cost does not depend on them)
    ks = n_sets(4 * n * 4)  # gate, up, dout read + out written per step
    ssets = [(gate0.clone().requires_grad_(True), up0.clone().requires_grad_(True), dout.clone())
             for _ in range(ks)]

    def step(i):
        gi, ui, di = ssets[i % ks]
        gi.grad = ui.grad = None
        swiglu(gi, ui).backward(di)

    ms, wall = sustained_steps(args, step)
    gbs = rate(bytes_step, ms, 1e9)
    cold = cold_figure(args, step, bytes_step)
    del ssets
    # dominant kernel: backward (5 tensor passes), sustained over rotating
    # sets of (gate, up, dout, out)
    bwd_bytes = 5 * n * 4
    k = n_sets(bwd_bytes)
    sets = [(gate0.clone(), up0.clone(), dout.clone(), torch.empty_like(gate0)) for _ in range(k)]
    st = L.stream_of(gate0)

    def bwd(i):
        gf, uf, df, _ = sets[i % k]
        L.forge_swiglu_bwd(0, df.data_ptr(), C, gf.data_ptr(), uf.data_ptr(), C, gf.data_ptr(), uf.data_ptr(), C,
                           R, C, 1.0, 1.0, st)

    def fwd(i):
        gf, uf, _, out = sets[i % k]
        L.forge_swiglu_fwd(0, gf.data_ptr(), uf.data_ptr(), C, out.data_ptr(), C, R, C, 1.0, 1.0, st)

    bwd_ms = time_sustained(bwd, max(args.steps, 20))
    fwd_ms = time_sustained(fwd, max(args.steps, 20))
    del sets
    res = {
        "config": {"workload": "swiglu_fwd_bwd", "dtype": "fp32", "shape": [R, C], "gate_multiplier": 1.0,
                   "down_multiplier": 1.0, "preserve_inputs": False},
        "value": gbs, "unit": "GB/s", "ms_per_step": rnd(ms, 5), "wall_ms_per_step": rnd(wall, 5),
        "frac_of_hbm_peak": rnd(gbs and gbs / HBM_PEAK_GBS, 4), "algorithmic_bytes_per_step": bytes_step,
        "timing": STEP_SUSTAINED_LABEL, "cold": cold, "launch_timing": SUSTAINED_LABEL,
        "launches_ms": {"forge_swiglu_fwd": round(fwd_ms, 5), "forge_swiglu_bwd": round(bwd_ms, 5)},
        "roofline": _roof("hbm", bwd_bytes / (bwd_ms * 1e-3) / 1e9, HBM_PEAK_GBS, "GB/s", _traffic("swiglu_bwd")),
        "copy_ceiling": copy_ceiling(args, bwd_bytes),
        "dtype": "f32",
    }
    if not (args.no_cpu_baseline or args.only_launches):
        from oracle.swiglu import swiglu_fwd_bwd

        rows = R  # the whole workload
        gc, uc, dc = gate0[:rows].cpu(), up0[:rows].cpu(), dout[:rows].cpu()
        t, reps = cpu_time(lambda: swiglu_fwd_bwd(gc, uc, dc))
        res["cpu_baseline"] = _cpu(8 * rows * C * 4 / t / 1e9, "GB/s",
                                   f"all {R} rows, reference torch path in fp32 + autograd, fwd+bwd, median of {reps}")
    return res


def _rope_inputs(B=4, S=4096, NQ=32, NKV=8, D=128):
    import torch
    from kernels.rope import rope_cos_sin

    g = torch.Generator(device="cuda").manual_seed(1)
    q = torch.randn(B, S, NQ, D, device="cuda", generator=g).to(torch.bfloat16)
    k = torch.randn(B, S, NKV, D, device="cuda", generator=g).to(torch.bfloat16)
    dq = torch.randn(B, S, NQ, D, device="cuda", generator=g).to(torch.bfloat16)
    dk = torch.randn(B, S, NKV, D, device="cuda", generator=g).to(torch.bfloat16)
    tabs = []
    for base in (10000.0, 500000.0):
        c, s = rope_cos_sin(torch.arange(S, device="cuda"), D, base, torch.bfloat16)
        tabs.append((c.unsqueeze(0), s.unsqueeze(0)))
    return q, k, dq, dk, tabs


def bench_rope(args):
    """bf16 Q [4,4096,32,128], K [4,4096,8,128] (B,S,H,D memory,
    passed as the HF transpose(1,2) view), bases 10000 and 500000."""
    import torch
    from forge_hip import _lib as L
    from kernels.rope import apply_rope
    from kernels.rope.forge_rope_v3 import _rope_launch

    B, S, NQ, NKV, D = 4, 4096, 32, 8, 128
    q, k, dq, dk, tabs = _rope_inputs(B, S, NQ, NKV, D)
    qv, kv = q.transpose(1, 2), k.transpose(1, 2)
    dqv, dkv = dq.transpose(1, 2), dk.transpose(1, 2)

    elems = q.numel() + k.numel()
    bytes_dir = 2 * elems * 2 + 2 * S * D * 2  # read+write Q,K + cos/sin (the reference's formula)
    bytes_step = 2 * bytes_dir
    # input sets (q, k, dq, dk) for the steps, HF transpose(1, 2) views of
    # BSHD memory; the base alternates
    ks = n_sets(bytes_step)
    ssets = [tuple(t.clone().transpose(1, 2) for t in (q, k, dq, dk)) for _ in range(ks)]

    def step(i):
        c, s = tabs[i % 2]
        qs, kss, dqs, dks = ssets[i % ks]
        qi = qs.detach().requires_grad_(True)
        ki = kss.detach().requires_grad_(True)
        oq, ok = apply_rope(qi, ki, c, s)
        torch.autograd.backward((oq, ok), (dqs, dks))

    ms, wall = sustained_steps(args, step)
    gbs = rate(bytes_step, ms, 1e9)
    cold = cold_figure(args, step, bytes_step)
    del ssets
    # one direction, sustained over rotating sets of (q, k, q_out, k_out),
    # each a fresh HF transpose(1, 2) view of BSHD memory; the base and the
    # direction alternate as in the steps
    nk = n_sets(bytes_dir)
    sets = []
    for _ in range(nk):
        qs, ks = q.clone().transpose(1, 2), k.clone().transpose(1, 2)
        sets.append((qs, ks, torch.empty_like(qs), torch.empty_like(ks)))

    def launch(i):
        qs, ks, oq, ok = sets[i % nk]
        _rope_launch(qs, ks, oq, ok, tabs[i % 2][0], tabs[i % 2][1], bool(i % 2))

    launch_ms = time_sustained(launch, max(2 * args.steps, 40))
    del sets
    res = {
        "config": {"workload": "rope_fwd_bwd", "dtype": "bf16", "q": [B, NQ, S, D], "k": [B, NKV, S, D],
                   "layout": "BSHD memory, HF transpose(1,2) view", "bases": [10000, 500000]},
        "value": gbs, "unit": "GB/s", "ms_per_step": rnd(ms, 5), "wall_ms_per_step": rnd(wall, 5),
        "frac_of_hbm_peak": rnd(gbs and gbs / HBM_PEAK_GBS, 4), "algorithmic_bytes_per_step": bytes_step,
        "timing": STEP_SUSTAINED_LABEL, "cold": cold, "launch_timing": SUSTAINED_LABEL,
        "launches_ms": {"forge_rope": round(launch_ms, 5)},
        "roofline": _roof("hbm", bytes_dir / (launch_ms * 1e-3) / 1e9, HBM_PEAK_GBS, "GB/s", _traffic("rope")),
        "copy_ceiling": copy_ceiling(args, bytes_dir),
        "dtype": "bf16",
    }
    if not (args.no_cpu_baseline or args.only_launches):
        from oracle.rope import rope_fwd_bwd

        sb = S  # all of batch 0: a quarter of the workload
        qc = q[:1, :sb].transpose(1, 2).cpu()
        kc = k[:1, :sb].transpose(1, 2).cpu()
        dqc, dkc = dq[:1, :sb].transpose(1, 2).cpu(), dk[:1, :sb].transpose(1, 2).cpu()
        c, s = tabs[0][0][:, :sb].cpu(), tabs[0][1][:, :sb].cpu()
        t, reps = cpu_time(lambda: rope_fwd_bwd(qc, kc, c, s, dqc, dkc))
        frac = sb / (B * S)
        res["cpu_baseline"] = _cpu(bytes_step * frac / t / 1e9, "GB/s",
                                   f"{sb} of {B * S} tokens (batch 0), HF formula in fp32 + autograd, fwd+bwd, "
                                   f"median of {reps}")
    return res


def bench_ce(args):
    """bf16 logits [8192, 128256] ~ N(0, 2^2), 5% ignore_index,
    mean reduction, grad_output = 1."""
    import torch
    from forge_hip import _lib as L
    from kernels.cross_entropy.experiments.v2 import forge_cross_entropy

    BT, V = 8192, 128256
    g = torch.Generator(device="cuda").manual_seed(2)
    logits0 = (torch.randn(BT, V, device="cuda", generator=g) * 2.0).to(torch.bfloat16)
    target = torch.randint(0, V, (BT,), device="cuda", generator=g)
    ign = torch.randperm(BT, device="cuda", generator=g)[:410]
    target[ign] = -100
    n_ign = 410
    n_valid = BT - n_ign
    xbuf = torch.empty_like(logits0)

    def restore(i):
        xbuf.copy_(logits0)  # the forward writes dlogits over the logits

    def step(i):
        x = xbuf.detach().requires_grad_(True)
        loss = forge_cross_entropy(x, target)
        loss.backward()

    ms, wall = run_steps(args, step, restore)
    bytes_step = V * 2 * (2 * n_valid + n_ign) + 8 * BT
    gbs = rate(bytes_step, ms, 1e9)
    # sustained over two 2.1 GB logits buffers (the steps' buffer and one
    # more): the forward's one launch, forge_ce_fwd_reduce (statistics, rows,
    # dlogits and the reduced loss)
    xbuf.copy_(logits0)
    xb = logits0.clone()
    sets = [xbuf, xb]
    loss1d = torch.empty(BT, device="cuda")
    lsum = torch.empty((), device="cuda")
    st = L.stream_of(xb)
    flags = L.CE_HAS_GRADIENTS | L.CE_REDUCTION_MEAN
    ticket = ctypes.c_uint64()
    launch_ms = time_sustained(
        lambda i: L.forge_ce_fwd_reduce(2, sets[i % 2].data_ptr(), V, BT, V, target.data_ptr(), 1, loss1d.data_ptr(),
                                        None, None, None, -100, 0.0, 0.0, 0.0, flags, lsum.data_ptr(), None, None,
                                        None, L.DTYPE_F32, ctypes.byref(ticket), st),
        max(args.steps, 20))
    del sets
    res = {
        "config": {"workload": "cross_entropy_fwd_bwd", "dtype": "bf16", "logits": [BT, V], "ignored_rows": n_ign,
                   "reduction": "mean", "grad_output": 1.0},
        "value": gbs, "unit": "GB/s", "ms_per_step": rnd(ms, 5), "wall_ms_per_step": rnd(wall, 5),
        "frac_of_hbm_peak": rnd(gbs and gbs / HBM_PEAK_GBS, 4), "algorithmic_bytes_per_step": bytes_step,
        "timing": "cold: each step alone after its logits are restored and a 512 MB read",
        "launch_timing": SUSTAINED_LABEL,
        "launches_ms": {"forge_ce_fwd_reduce": round(launch_ms, 5)},
        "launches_per_step": "forward: forge_ce_fwd_reduce (1); backward: forge_ce_scale, a no-op on the device "
                             "for grad_output == 1 (1), after torch's implicit ones_like for loss.backward()",
        "roofline": _roof("hbm", bytes_step / (launch_ms * 1e-3) / 1e9, HBM_PEAK_GBS, "GB/s", _traffic("ce_fwd")),
        "copy_ceiling": None,
        "dtype": "bf16",
    }
    del xb
    res["copy_ceiling"] = copy_ceiling(args, bytes_step)
    if not (args.no_cpu_baseline or args.only_launches):
        import torch.nn.functional as F

        rows = 1024
        xc = logits0[:rows].cpu()
        tc = target[:rows].cpu()

        def cpu_step():
            x = xc.clone().requires_grad_(True)
            F.cross_entropy(x, tc, ignore_index=-100).backward()

        t, reps = cpu_time(cpu_step)
        nv = int((tc != -100).sum())
        res["cpu_baseline"] = _cpu((V * 2 * (2 * nv + (rows - nv)) + 8 * rows) / t / 1e9, "GB/s",
                                   f"{rows} of {BT} rows, F.cross_entropy (the reference's CPU path) bf16 fwd+bwd, "
                                   f"median of {reps}")
    return res


def _gpu_params_mlp(H, I, r, alpha, gen):
    """configs[3] initialisation on the GPU (same distributions as
    oracle/lora_mlp.py make_params)."""
    import torch

    s = alpha / r
    bf = torch.bfloat16

    def W(o, i):
        return (torch.randn(o, i, device="cuda", generator=gen) * 0.02).to(bf)

    def A(i):
        return ((torch.rand(r, i, device="cuda", generator=gen) * 2 - 1) / i ** 0.5).to(bf).requires_grad_(True)

    def B(o):
        return (torch.randn(o, r, device="cuda", generator=gen) * 0.01).to(bf).requires_grad_(True)

    return (W(I, H), A(H), B(I), s, W(I, H), A(H), B(I), s, W(H, I), A(I), B(H), s)


def _hipblaslt_leg(args, M, N, K, flops_, seed=12):
    """Comparison leg, not the product: hipBLASLt (torch.matmul) on a plain
    bf16 product of the same FLOPs as the step's dominant library launch,
    timed the same way (cold launches), so the library GEMM can be judged
    against the vendor library on this box."""
    import torch

    bf = torch.bfloat16
    g = torch.Generator(device="cuda").manual_seed(seed)
    A = torch.randn(M, K, device="cuda", generator=g).to(bf)
    B = (torch.randn(N, K, device="cuda", generator=g) * 0.02).to(bf)
    C = torch.empty(M, N, device="cuda", dtype=bf)
    ms = time_launches(lambda i: torch.matmul(A, B.t(), out=C), max(args.steps, 10))
    del A, B, C
    return {"what": f"hipBLASLt torch.matmul {M} x {N} x {K} (plain, no epilogue)", "ms": round(ms, 4),
            "tflops": round(flops_ / (ms * 1e-3) / 1e12, 1)}


def _gate_up_roofline(args, M, H, I, r, Wg, Wu, traffic_key="lora_mlp_gate_up", activation=None):
    """(label, mean launch ms, roofline, hipBLASLt comparison) of the LoRA-MLP
    step's largest launch: forge_lora_mlp_gate_up, the dual gate/up GEMM with
    the LoRA-B products as K segments and the gated activation in its
    epilogue (e, g, h stored), as the step issues it."""
    import torch
    from forge_hip import _lib as L

    bf = torch.bfloat16
    act = L.ACT_SILU if activation is None else activation
    g = torch.Generator(device="cuda").manual_seed(11)
    X = torch.randn(M, H, device="cuda", generator=g).to(bf)
    xa = (torch.randn(M, 2 * r, device="cuda", generator=g) * 0.1).to(bf)
    Bg = (torch.randn(I, r, device="cuda", generator=g) * 0.01).to(bf)
    Bu = (torch.randn(I, r, device="cuda", generator=g) * 0.01).to(bf)
    e = torch.empty(M, I, dtype=bf, device="cuda")
    gg = torch.empty_like(e)
    h = torch.empty_like(e)
    st = L.stream_of(X)

    def launch(i):
        L.check(L.forge_lora_mlp_gate_up(M, H, I, r, X.data_ptr(), H, Wg.data_ptr(), Wu.data_ptr(), Wg.stride(0),
                                         xa.data_ptr(), 2 * r, Bg.data_ptr(), Bu.data_ptr(), r, e.data_ptr(),
                                         gg.data_ptr(), h.data_ptr(), I, act, st), "forge_lora_mlp_gate_up")

    launch_ms = time_launches(launch, max(args.steps, 10))
    del X, xa, e, gg, h
    fl = 4 * M * H * I + 4 * M * r * I
    label = f"forge_lora_mlp_gate_up (dual gate/up GEMM + GLU epilogue, {M} x {2 * I} x {H} + LoRA-B segments)"
    cmp_ = _hipblaslt_leg(args, M, 2 * I, H, 4 * M * H * I)
    return label, launch_ms, _roof("mfma", fl / (launch_ms * 1e-3) / 1e12, BF16_PEAK_TFLOPS, "TFLOP/s",
                                   _traffic(traffic_key)), cmp_


def bench_lora_mlp(args, activation="silu"):
    """LoRA MLP fwd+bwd, bf16, Llama-3-8B shape (M=8192, H=4096,
    I=14336), r=16, alpha=32.  activation="gelu_tanh" runs the fused
    LoRA-GeGLU MLP (LoRAMLPGeGLU, Gemma's activation) on the same shape."""
    import torch
    from forge_hip import _lib as L
    from kernels.lora_mlp.experiments.v6.lora_mlp_kernel_v6 import LoRAMLPv6
    from kernels.lora_mlp.geglu_mlp import LoRAMLPGeGLU
    from oracle.lora_mlp import flops

    geglu = activation != "silu"
    M, H, I, r = 8192, 4096, 14336, 16
    g = torch.Generator(device="cuda").manual_seed(3)
    params = _gpu_params_mlp(H, I, r, 32, g)
    X = torch.randn(1, M, H, device="cuda", generator=g).to(torch.bfloat16).requires_grad_(True)
    dY = torch.randn(1, M, H, device="cuda", generator=g).to(torch.bfloat16)

    leaves = [X] + [t for t in params if isinstance(t, torch.Tensor) and t.requires_grad]

    def step(i):
        for t in leaves:  # a training step after zero_grad(set_to_none=True)
            t.grad = None
        out = LoRAMLPGeGLU.apply(X, *params, "tanh") if geglu else LoRAMLPv6.apply(X, *params)
        out.backward(dY)

    ms, wall = run_steps(args, step)
    fl = flops(M, H, I, r)
    tf = rate(fl, ms, 1e12)
    # roofline kernel: the step's largest launch, the fused gate/up GEMM
    label, launch_ms, roof, cmp_ = _gate_up_roofline(
        args, M, H, I, r, params[0].detach(), params[4].detach(),
        traffic_key="lora_mlp_geglu_gate_up" if geglu else "lora_mlp_gate_up",
        activation=L.ACT_GELU_TANH if geglu else L.ACT_SILU)
    res = {
        "config": {"workload": "lora_mlp_geglu_fwd_bwd" if geglu else "lora_mlp_fwd_bwd", "dtype": "bf16", "M": M,
                   "H": H, "I": I, "rank": r, "alpha": 32,
                   "api": "LoRAMLPGeGLU (tanh GELU)" if geglu else "LoRAMLPv6"},
        "value": tf, "unit": "TFLOP/s", "ms_per_step": rnd(ms, 4), "wall_ms_per_step": rnd(wall, 4),
        "frac_of_mfma_peak": rnd(tf and tf / BF16_PEAK_TFLOPS, 4), "algorithmic_flops_per_step": fl,
        "launches_ms": {label: round(launch_ms, 4)},
        "roofline": roof,
        "comparison_hipblaslt": cmp_,
        "dtype": "bf16",
    }
    if not (args.no_cpu_baseline or args.only_launches):
        from oracle.lora_mlp import fwd_bwd

        ms_ = 512
        cpu_params = [t.detach().cpu() if isinstance(t, torch.Tensor) else t for t in params]
        Xc, dYc = X.detach()[:, :ms_].cpu(), dY[:, :ms_].cpu()
        t, reps = cpu_time(lambda: fwd_bwd(Xc, dYc, cpu_params, compute_dtype=torch.bfloat16, activation=activation))
        what = ("the reference's Gemma composition (LoRA projections + GeGLU)" if geglu
                else "reference LoRAMLP formulas")
        res["cpu_baseline"] = _cpu(flops(ms_, H, I, r) / t / 1e12, "TFLOP/s",
                                   f"{ms_} of {M} tokens, {what} in bf16, fwd+bwd, median of {reps}")
    return res


def bench_lora_mlp_geglu(args):
    return bench_lora_mlp(args, activation="gelu_tanh")


class _PeftLayoutLoRA:
    """Builds an nn.Module with peft.tuners.lora.Linear's attributes and
    forward (base_layer, lora_A / lora_B ModuleDicts, scaling, lora_dropout,
    active_adapters; base(x) + lora_B(lora_A(x)) * scaling): peft itself is
    not installed on these boxes."""

    @staticmethod
    def wrap(base, r, alpha, gen):
        import torch
        import torch.nn as nn

        class LoraLinear(nn.Module):
            def __init__(self):
                super().__init__()
                self.base_layer = base
                dev, dt = base.weight.device, base.weight.dtype
                self.lora_A = nn.ModuleDict({"default": nn.Linear(base.in_features, r, bias=False, device=dev, dtype=dt)})
                self.lora_B = nn.ModuleDict({"default": nn.Linear(r, base.out_features, bias=False, device=dev, dtype=dt)})
                with torch.no_grad():
                    self.lora_A["default"].weight.copy_(torch.randn(r, base.in_features, generator=gen, device=dev)
                                                        / base.in_features ** 0.5)
                    self.lora_B["default"].weight.copy_(torch.randn(base.out_features, r, generator=gen, device=dev)
                                                        * 0.01)
                self.lora_dropout = nn.ModuleDict({"default": nn.Identity()})
                self.scaling = {"default": alpha / r}
                self.active_adapters = ["default"]
                self.disable_adapters = False
                self.merged = False
                base.weight.requires_grad_(False)

            def forward(self, x):
                a, b = self.lora_A["default"], self.lora_B["default"]
                return self.base_layer(x) + b(a(x)) * self.scaling["default"]

        return LoraLinear()


def bench_lora_patch(args, arch="llama"):
    """The patch-layer adapter (forge/patching/kernels/lora.py) on Hugging
    Face's LlamaMLP at the LoRA-MLP config (M=8192, H=4096, I=14336, r=16,
    alpha=32), PEFT-layout LoRA on gate/up/down, fwd+bwd: the fused adapter
    against the reference adapter's submodule path (PEFT projections on
    hipBLASLt GEMMs + the SwiGLU kernel) on the same module and inputs.
    arch="gemma2": Gemma2MLP at Gemma-2-9B's MLP shape (H=3584, I=14336,
    tanh GELU), the fused LoRA-GeGLU MLP against the reference's Gemma path
    (PEFT projections + the GeGLU kernel, lora.py:184-188)."""
    import copy

    import torch

    try:
        from transformers import Gemma2Config, LlamaConfig
        import transformers.models.gemma2.modeling_gemma2 as MG
        import transformers.models.llama.modeling_llama as ML
    except ImportError:
        return {"skipped": "transformers is not installed", "value": None, "unit": "TFLOP/s"}
    from forge.patching import FORWARD_MAKERS
    from forge.kernels.geglu import geglu
    from forge.kernels.swiglu import swiglu
    from forge_hip import _lib as L
    from oracle.lora_mlp import flops

    gemma = arch == "gemma2"
    M, H, I, r = (8192, 3584, 14336, 16) if gemma else (8192, 4096, 14336, 16)
    g = torch.Generator(device="cuda").manual_seed(9)
    torch.manual_seed(9)
    if gemma:
        cfg = Gemma2Config(hidden_size=H, intermediate_size=I, num_attention_heads=16, num_key_value_heads=8,
                           head_dim=256, hidden_activation="gelu_pytorch_tanh")
        ref = MG.Gemma2MLP(cfg).to("cuda", torch.bfloat16)
    else:
        cfg = LlamaConfig(hidden_size=H, intermediate_size=I, num_attention_heads=32, num_key_value_heads=8,
                          head_dim=128)
        ref = ML.LlamaMLP(cfg).to("cuda", torch.bfloat16)
    for n in ("gate_proj", "up_proj", "down_proj"):
        setattr(ref, n, _PeftLayoutLoRA.wrap(getattr(ref, n), r, 32, g))
    fused = copy.deepcopy(ref)
    fused.forward = FORWARD_MAKERS["lora_mlp"](fused, {})
    if gemma:
        # the reference adapter's Gemma path (lora.py:184-188): PEFT submodules + geglu
        ref.forward = lambda x: ref.down_proj(geglu(ref.gate_proj(x), ref.up_proj(x), approximate="tanh"))
    else:
        # the reference adapter's call path (lora.py:160-163): PEFT submodules + swiglu
        ref.forward = lambda x: ref.down_proj(swiglu(ref.gate_proj(x), ref.up_proj(x)))
    X = torch.randn(1, M, H, device="cuda", generator=g).to(torch.bfloat16).requires_grad_(True)
    dY = torch.randn(1, M, H, device="cuda", generator=g).to(torch.bfloat16)

    def stepper(mod):
        leaves = [X] + [p for p in mod.parameters() if p.requires_grad]

        def step(i):
            for t in leaves:
                t.grad = None
            mod(X).backward(dY)
        return step

    ms, wall = run_steps(args, stepper(fused))
    ms_ref, _ = run_steps(args, stepper(ref))
    fl = flops(M, H, I, r)
    tf, tf_ref = rate(fl, ms, 1e12), rate(fl, ms_ref, 1e12)
    label, launch_ms, roof, cmp_ = _gate_up_roofline(
        args, M, H, I, r, ref.gate_proj.base_layer.weight.detach(), ref.up_proj.base_layer.weight.detach(),
        traffic_key="lora_patch_gemma_gate_up" if gemma else "lora_mlp_gate_up",
        activation=L.ACT_GELU_TANH if gemma else L.ACT_SILU)
    return {
        "config": {"workload": "lora_mlp_patch_gemma2_fwd_bwd" if gemma else "lora_mlp_patch_fwd_bwd", "dtype": "bf16",
                   "M": M, "H": H, "I": I, "rank": r, "alpha": 32,
                   "module": f"transformers {'Gemma2MLP (tanh GELU)' if gemma else 'LlamaMLP'}, PEFT-layout LoRA on "
                             "gate/up/down",
                   "api": "forge.patching FORWARD_MAKERS['lora_mlp']"},
        "value": tf, "unit": "TFLOP/s", "ms_per_step": rnd(ms, 4), "wall_ms_per_step": rnd(wall, 4),
        "frac_of_mfma_peak": rnd(tf and tf / BF16_PEAK_TFLOPS, 4), "algorithmic_flops_per_step": fl,
        "reference_submodule_path": {"value": tf_ref, "unit": "TFLOP/s", "ms_per_step": rnd(ms_ref, 4)},
        "speedup_vs_submodule_path": rnd(ms and ms_ref / ms, 3),
        "launches_ms": {label: round(launch_ms, 4)},
        "roofline": roof,
        "comparison_hipblaslt": cmp_,
        "dtype": "bf16",
    }


def bench_lora_patch_gemma(args):
    return bench_lora_patch(args, arch="gemma2")


def bench_lora_qkv(args):
    """fused LoRA QKV (GQA 32/8, head_dim 128, hidden 4096, r=64,
    alpha=128) then RoPE (base 500000), 8 varlen sequences U[512, 4096]."""
    import torch
    from kernels.lora_qkv.experiments.v4.lora_qkv_kernel_v4 import lora_qkv_rope
    from kernels.rope import rope_cos_sin
    from oracle.lora_qkv import flops_per_token, positions_for, varlen_lengths

    K, Hq, Hkv, D, r = 4096, 4096, 1024, 128, 64
    lens = varlen_lengths(8, 512, 4096, seed=4)
    pos = positions_for(lens).cuda()
    T = int(pos.numel())
    g = torch.Generator(device="cuda").manual_seed(4)
    bf = torch.bfloat16

    def W(o):
        return (torch.randn(o, K, device="cuda", generator=g) * 0.02).to(bf)

    def A():
        return ((torch.rand(r, K, device="cuda", generator=g) * 2 - 1) / K ** 0.5).to(bf).requires_grad_(True)

    def B(o):
        return (torch.randn(o, r, device="cuda", generator=g) * 0.01).to(bf).requires_grad_(True)

    s = 128 / r
    Wq, Wk, Wv = W(Hq), W(Hkv), W(Hkv)
    Aq, Bq, Ak, Bk, Av, Bv = A(), B(Hq), A(), B(Hkv), A(), B(Hkv)
    X = torch.randn(T, K, device="cuda", generator=g).to(bf).requires_grad_(True)
    dQ = torch.randn(T, Hq, device="cuda", generator=g).to(bf)
    dK = torch.randn(T, Hkv, device="cuda", generator=g).to(bf)
    dV = torch.randn(T, Hkv, device="cuda", generator=g).to(bf)
    c, sn = rope_cos_sin(torch.arange(max(lens), device="cuda"), D, 500000.0, bf)

    leaves = (X, Aq, Bq, Ak, Bk, Av, Bv)

    def step(i):
        for t in leaves:  # a training step after zero_grad(set_to_none=True)
            t.grad = None
        Q, K_, V = lora_qkv_rope(X, Wq, Aq, Bq, s, Wk, Ak, Bk, s, Wv, Av, Bv, s, c, sn, pos, D)
        torch.autograd.backward((Q, K_, V), (dQ, dK, dV))

    ms, wall = run_steps(args, step)
    fl = T * flops_per_token(K, Hq, Hkv, r)
    tf = rate(fl, ms, 1e12)
    # dominant kernel: the forward product, forge_lora_qkv_rope (X [Wq;Wk;Wv]^T
    # with the LoRA-B products as K segments and RoPE in its epilogue); the
    # backward's dX product is the other one of its size
    from kernels._lora_ops import lora_a
    from kernels.lora_qkv._impl import qkv_gemm

    Xd = X.detach()
    xa = lora_a(Xd, [Aq.detach(), Ak.detach(), Av.detach()], [s, s, s])  # the forward's LoRA-A product
    out = torch.empty(T, Hq + 2 * Hkv, device="cuda", dtype=bf)
    rope = {"cos": c, "sin": sn, "positions": pos, "head_dim": D}
    launch_ms = time_launches(lambda i: qkv_gemm(Xd, Wq, Wk, Wv, xa, Bq.detach(), Bk.detach(), Bv.detach(), r,
                                                 rope, out), max(args.steps, 10))
    del out
    fwd_flops = 2 * T * K * (Hq + 2 * Hkv) + 2 * T * r * (Hq + 2 * Hkv)
    res = {
        "config": {"workload": "lora_qkv_rope_fwd_bwd", "dtype": "bf16", "tokens": T, "seq_lens": lens,
                   "hidden": K, "q_heads": 32, "kv_heads": 8, "head_dim": D, "rank": r, "alpha": 128,
                   "rope_base": 500000},
        "value": tf, "unit": "TFLOP/s", "ms_per_step": rnd(ms, 4), "wall_ms_per_step": rnd(wall, 4),
        "frac_of_mfma_peak": rnd(tf and tf / BF16_PEAK_TFLOPS, 4), "algorithmic_flops_per_step": fl,
        "launches_ms": {f"forge_lora_qkv_rope (QKV GEMM + LoRA-B segments + RoPE epilogue, {T} x "
                        f"{Hq + 2 * Hkv} x {K})": round(launch_ms, 4)},
        "roofline": _roof("mfma", fwd_flops / (launch_ms * 1e-3) / 1e12, BF16_PEAK_TFLOPS, "TFLOP/s",
                          _traffic("lora_qkv_fwd_gemm")),
        "comparison_hipblaslt": _hipblaslt_leg(args, T, Hq + 2 * Hkv, K, 2 * T * K * (Hq + 2 * Hkv)),
        "dtype": "bf16",
    }
    if not (args.no_cpu_baseline or args.only_launches):
        from oracle.lora_qkv import qkv_rope_fwd_bwd

        n = 1024
        cpu_p = [t.detach().cpu() if isinstance(t, torch.Tensor) else t
                 for t in (Wq, Wk, Wv, Aq, Bq, s, Ak, Bk, s, Av, Bv, s)]
        pc = pos[:n].cpu()
        args_ = (X.detach()[:n].cpu(), dQ[:n].cpu(), dK[:n].cpu(), dV[:n].cpu(), cpu_p, c.cpu()[pc], sn.cpu()[pc], D)
        t, reps = cpu_time(lambda: qkv_rope_fwd_bwd(*args_, compute_dtype=torch.bfloat16))
        res["cpu_baseline"] = _cpu(n * flops_per_token(K, Hq, Hkv, r) / t / 1e12, "TFLOP/s",
                                   f"{n} of {T} tokens, reference LoRAQKV + HF RoPE in bf16, fwd+bwd, median of {reps}")
    return res


def _roof(bound, achieved, peak, unit, traffic):
    return {"bound": bound, "achieved": round(achieved, 2), "peak": peak, "unit": unit,
            "frac": round(achieved / peak, 4), "traffic": traffic}


def _cpu(value, unit, sample):
    import torch

    return {"value": round(value, 3), "unit": unit, "cores": torch.get_num_threads(), "kind": "port",
            "sample": sample, "cpu_count": os.cpu_count()}


def bench_copy(args):
    """Calibration workload for the rocprofv3 byte counters: forge_cast_f32_bf16
    over 2^28 fp32 values reads exactly 1 GiB and writes exactly 512 MiB, so
    FETCH_SIZE / WRITE_SIZE of its dispatches give the counters' scale."""
    import torch
    from forge_hip import _lib as L

    n = 1 << 28
    src = torch.randn(n, device="cuda")
    dst = torch.empty(n, device="cuda", dtype=torch.bfloat16)
    st = L.stream_of(src)
    ms = time_launches(lambda i: L.forge_cast_f32_bf16(src.data_ptr(), n, dst.data_ptr(), n, 1, n, st),
                       max(args.steps, 10))
    moved = n * 4 + n * 2
    gbs = moved / (ms * 1e-3) / 1e9
    return {"config": {"workload": "copy_calibration", "read_bytes": n * 4, "write_bytes": n * 2},
            "value": round(gbs, 1), "unit": "GB/s", "ms_per_step": round(ms, 5), "launches_ms":
            {"forge_cast_f32_bf16": round(ms, 5)}, "roofline": _roof("hbm", gbs, HBM_PEAK_GBS, "GB/s", None),
            "dtype": "f32"}


def bench_flce(args):
    """Fused linear + cross-entropy (the next row after the five configs): the
    Llama-3-8B lm_head shape, bf16 hidden [8192, 4096] and weight
    [128256, 4096], 5% ignore_index, mean, fwd+bwd with input and weight
    gradients."""
    import torch
    from forge_hip import _lib as L
    from kernels.cross_entropy.experiments.v2 import forge_fused_linear_cross_entropy
    from oracle.fused_linear_ce import flops

    BT, H, V = 8192, 4096, 128256
    bf = torch.bfloat16
    g = torch.Generator(device="cuda").manual_seed(6)
    x = torch.randn(BT, H, device="cuda", generator=g).to(bf).requires_grad_(True)
    W = (torch.randn(V, H, device="cuda", generator=g) / H ** 0.5).to(bf).requires_grad_(True)
    target = torch.randint(0, V, (BT,), device="cuda", generator=g)
    target[torch.randperm(BT, device="cuda", generator=g)[:410]] = -100

    def step(i):
        x.grad = None  # a training step after zero_grad(set_to_none=True)
        W.grad = None
        forge_fused_linear_cross_entropy(x, W, target).backward()

    ms, wall = run_steps(args, step)
    fl = flops(BT, H, V)
    tf = rate(fl, ms, 1e12)
    # dominant kernel: the library GEMM that computes the logits of one chunk
    # (X_c W^T; at this shape the whole batch is one 2 GiB chunk); dX_c =
    # dlogits W and dW are the same size
    from kernels._lora_ops import COL, ROW, gemm
    from kernels.cross_entropy.experiments.v2.fused_linear_cross_entropy import _chunk_rows
    n = _chunk_rows(BT, V * 2)
    logits = torch.empty(n, V, device="cuda", dtype=bf)
    xc, wd = x.detach()[:n], W.detach()
    launch_ms = time_launches(lambda i: gemm(n, V, [(xc, H, wd, H, H)], ROW, COL, out=logits), max(args.steps, 10))
    del logits
    res = {
        "config": {"workload": "fused_linear_cross_entropy_fwd_bwd", "dtype": "bf16", "tokens": BT, "hidden": H,
                   "vocab": V, "ignored_rows": 410, "reduction": "mean", "chunk_tokens": n,
                   "api": "forge_fused_linear_cross_entropy"},
        "value": tf, "unit": "TFLOP/s", "ms_per_step": rnd(ms, 4), "wall_ms_per_step": rnd(wall, 4),
        "frac_of_mfma_peak": rnd(tf and tf / BF16_PEAK_TFLOPS, 4), "algorithmic_flops_per_step": fl,
        "launches_ms": {f"forge_gemm logits GEMM (X_c W^T, {n} x {V} x {H})": round(launch_ms, 4)},
        "roofline": _roof("mfma", 2 * n * H * V / (launch_ms * 1e-3) / 1e12, BF16_PEAK_TFLOPS, "TFLOP/s",
                          _traffic("flce_logits_gemm")),
        "comparison_hipblaslt": _hipblaslt_leg(args, n, V, H, 2 * n * H * V),
        "dtype": "bf16",
    }
    if not (args.no_cpu_baseline or args.only_launches):
        from oracle.fused_linear_ce import fused_linear_ce

        rows = 64
        xc_cpu, wc, tc = x.detach()[:rows].float().cpu(), W.detach().float().cpu(), target[:rows].cpu()
        t, reps = cpu_time(lambda: fused_linear_ce(xc_cpu, wc, tc, compute_dtype=torch.float32))
        res["cpu_baseline"] = _cpu(flops(rows, H, V) / t / 1e12, "TFLOP/s",
                                   f"{rows} of {BT} tokens, the reference's linear + CE formulas in fp32 "
                                   f"(torch CPU matmuls), fwd+bwd, median of {reps}")
    return res


def bench_geglu(args):
    """GeGLU (the next row after the five configs): the Gemma-7B MLP shape,
    bf16 gate/up/dout [4096, 24576], tanh GELU, out = gelu(gate) * up."""
    import torch
    from forge_hip import _lib as L
    from kernels.geglu import geglu

    R, C = 4096, 24576
    n = R * C
    bf = torch.bfloat16
    g = torch.Generator(device="cuda").manual_seed(7)
    gate0 = torch.randn(R, C, device="cuda", generator=g).to(bf)
    up0 = torch.randn(R, C, device="cuda", generator=g).to(bf)
    dout = torch.randn(R, C, device="cuda", generator=g).to(bf)
    bytes_step = 8 * n * 2  # fwd 3 tensors + bwd 5 tensors, bf16
    # input sets (gate, up, dout); the backward's in-place gradients become
    # the set's next inputs (finite; the cost does not depend on the values)
    ks = n_sets(4 * n * 2)
    ssets = [(gate0.clone().requires_grad_(True), up0.clone().requires_grad_(True), dout.clone())
             for _ in range(ks)]

    def step(i):
        gi, ui, di = ssets[i % ks]
        gi.grad = ui.grad = None
        geglu(gi, ui, "tanh").backward(di)

    ms, wall = sustained_steps(args, step)
    gbs = rate(bytes_step, ms, 1e9)
    cold = cold_figure(args, step, bytes_step)
    del ssets
    # the backward, sustained over rotating sets of (gate, up, dout)
    k = n_sets(5 * n * 2)
    sets = [(gate0.clone(), up0.clone(), dout.clone()) for _ in range(k)]
    st = L.stream_of(gate0)

    def bwd(i):
        gf, uf, df = sets[i % k]
        L.forge_geglu_bwd(2, df.data_ptr(), C, gf.data_ptr(), uf.data_ptr(), C, gf.data_ptr(), uf.data_ptr(), C,
                          R, C, 1, st)

    bwd_ms = time_sustained(bwd, max(args.steps, 20))
    del sets
    res = {
        "config": {"workload": "geglu_fwd_bwd", "dtype": "bf16", "shape": [R, C], "approximate": "tanh"},
        "value": gbs, "unit": "GB/s", "ms_per_step": rnd(ms, 5), "wall_ms_per_step": rnd(wall, 5),
        "frac_of_hbm_peak": rnd(gbs and gbs / HBM_PEAK_GBS, 4), "algorithmic_bytes_per_step": bytes_step,
        "timing": STEP_SUSTAINED_LABEL, "cold": cold, "launch_timing": SUSTAINED_LABEL,
        "launches_ms": {"forge_geglu_bwd": round(bwd_ms, 5)},
        "roofline": _roof("hbm", 5 * n * 2 / (bwd_ms * 1e-3) / 1e9, HBM_PEAK_GBS, "GB/s", _traffic("geglu_bwd")),
        "copy_ceiling": copy_ceiling(args, 5 * n * 2),
        "dtype": "bf16",
    }
    if not (args.no_cpu_baseline or args.only_launches):
        from oracle.geglu import geglu_fwd_bwd

        rows = 256
        gc, uc, dc = gate0[:rows].cpu(), up0[:rows].cpu(), dout[:rows].cpu()
        t, reps = cpu_time(lambda: geglu_fwd_bwd(gc, uc, dc, "tanh"))
        res["cpu_baseline"] = _cpu(8 * rows * C * 2 / t / 1e9, "GB/s",
                                   f"{rows} of {R} rows, the reference's GeGLU formulas (float64 torch), fwd+bwd, "
                                   f"median of {reps}")
    return res


def bench_rmsnorm(args):
    """RMSNorm (the next row after the five configs): bf16 x [8192, 4096]
    (Llama-3-8B hidden size), llama casting, fwd+bwd with the weight
    gradient and the in-place dY -> dX backward (v4 default)."""
    import torch
    from forge_hip import _lib as L
    from kernels.rmsnorm import apply_rmsnorm_v4
    from oracle.rmsnorm import bytes_fwd_bwd

    R, H = 8192, 4096
    bf = torch.bfloat16
    g = torch.Generator(device="cuda").manual_seed(8)
    x = torch.randn(R, H, device="cuda", generator=g).to(bf).requires_grad_(True)
    w = (1 + 0.1 * torch.randn(H, device="cuda", generator=g)).to(bf).requires_grad_(True)
    dy0 = torch.randn(R, H, device="cuda", generator=g).to(bf)
    bytes_step = bytes_fwd_bwd(R, H)
    # input sets (x, dy); the in-place backward writes dx over dy, which the
    # set's next step takes as its upstream gradient
    ks = n_sets(3 * R * H * 2)  # x, dy read + y written per step
    ssets = [(x.detach().clone().requires_grad_(True), dy0.clone()) for _ in range(ks)]

    def step(i):
        xs, dys = ssets[i % ks]
        xs.grad = None  # a training step after zero_grad(set_to_none=True)
        w.grad = None
        apply_rmsnorm_v4(xs, w, 1e-6, 0.0, "llama", in_place=True).backward(dys)

    ms, wall = sustained_steps(args, step)
    gbs = rate(bytes_step, ms, 1e9)
    cold = cold_figure(args, step, bytes_step)
    del ssets
    # dominant kernel: the backward (reads x and dy, writes dx over dy, dw partials)
    xd, wd = x.detach(), w.detach()
    rstd = torch.empty(R, device="cuda")
    yb = torch.empty_like(xd)
    st = L.stream_of(xd)
    L.check(L.forge_rmsnorm_fwd(2, 2, 2, xd.data_ptr(), H, wd.data_ptr(), yb.data_ptr(), H, rstd.data_ptr(), R, H,
                                1e-6, 0.0, 0, st), "forge_rmsnorm_fwd")
    bwd_bytes = 3 * R * H * 2 + 4 * R + 3 * H * 2
    # sustained over rotating sets of (x, dy, dx) (rstd and the weight are shared)
    k = n_sets(bwd_bytes)
    sets = [(xd.clone(), dy0.clone(), torch.empty_like(xd)) for _ in range(k)]
    dw = torch.empty(H, device="cuda", dtype=bf)
    work = torch.empty(L.forge_rmsnorm_bwd_workspace(2, R, H), device="cuda", dtype=torch.uint8)

    def bwd(i):
        xs, dys, dxs = sets[i % k]
        L.forge_rmsnorm_bwd(2, 2, dys.data_ptr(), H, xs.data_ptr(), H, wd.data_ptr(), rstd.data_ptr(), dxs.data_ptr(),
                            H, dw.data_ptr(), work.data_ptr(), R, H, 0.0, 0, st)

    bwd_ms = time_sustained(bwd, max(args.steps, 20))
    del sets
    res = {
        "config": {"workload": "rmsnorm_fwd_bwd", "dtype": "bf16", "shape": [R, H], "casting_mode": "llama",
                   "offset": 0.0, "in_place": True, "weight_grad": True},
        "value": gbs, "unit": "GB/s", "ms_per_step": rnd(ms, 5), "wall_ms_per_step": rnd(wall, 5),
        "frac_of_hbm_peak": rnd(gbs and gbs / HBM_PEAK_GBS, 4), "algorithmic_bytes_per_step": bytes_step,
        "timing": STEP_SUSTAINED_LABEL, "cold": cold, "launch_timing": SUSTAINED_LABEL,
        "launches_ms": {"forge_rmsnorm_bwd": round(bwd_ms, 5)},
        "roofline": _roof("hbm", bwd_bytes / (bwd_ms * 1e-3) / 1e9, HBM_PEAK_GBS, "GB/s", _traffic("rmsnorm_bwd")),
        "copy_ceiling": copy_ceiling(args, bwd_bytes),
        "dtype": "bf16",
    }
    if not (args.no_cpu_baseline or args.only_launches):
        from kernels.rmsnorm import torch_rmsnorm_reference_v4

        rows = 512
        xc = xd[:rows].cpu().requires_grad_(True)
        wc = wd.cpu().requires_grad_(True)
        gc = dy0[:rows].cpu()

        def cpu_step():
            xc.grad = None
            wc.grad = None
            torch_rmsnorm_reference_v4(xc, wc, 1e-6, 0.0, "llama").backward(gc)

        t, reps = cpu_time(cpu_step)
        res["cpu_baseline"] = _cpu(bytes_fwd_bwd(rows, H) / t / 1e9, "GB/s",
                                   f"{rows} of {R} rows, the reference's PyTorch RMSNorm (bf16) fwd+bwd via "
                                   f"autograd, median of {reps}")
    return res


BENCHES = {"copy": bench_copy, "swiglu": bench_swiglu, "rope": bench_rope, "ce": bench_ce, "lora_mlp": bench_lora_mlp,
           "lora_mlp_geglu": bench_lora_mlp_geglu, "lora_patch_gemma": bench_lora_patch_gemma, "lora_qkv": bench_lora_qkv, "flce": bench_flce, "geglu": bench_geglu,
           "rmsnorm": bench_rmsnorm, "lora_patch": bench_lora_patch}


def main():
    args = _parse()
    if args.gpus != 1:
        print(json.dumps({"error": f"--gpus {args.gpus}: this build measures one GPU only (single-GPU box); "
                                   "multi-GPU sharding is designed, not run here"}))
        return 2
    import torch

    if not torch.cuda.is_available():
        print(json.dumps({"error": "no ROCm GPU visible"}))
        return 1
    # the host share this process may use (OMP_NUM_THREADS on the GPU box), else every core
    torch.set_num_threads(int(os.environ.get("OMP_NUM_THREADS", 0)) or os.cpu_count() or 1)
    names = [n for n in args.kernels.split(",") if n]
    results = {}
    for n in names:
        fn = BENCHES.get(n)
        if fn is None:
            continue
        print(f"[bench] {n} ...", file=sys.stderr, flush=True)
        results[n] = fn(args)
        torch.cuda.empty_cache()
        print(f"[bench] {n}: {results[n]['value']} {results[n]['unit']}", file=sys.stderr, flush=True)
    head = results.get("rope") or next((r for r in results.values() if r.get("roofline")), None)
    if head is None:
        print(json.dumps({"error": "no timed workload", "kernels": results}))
        return 1
    line = {
        "metric": METRIC,
        "value": head["value"],
        "unit": head["unit"],
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": head["dtype"],
        "data": "synthetic",
        "config": head["config"],
        "timing": head.get("timing"),
        "cold": head.get("cold"),
        "roofline": head["roofline"],
        "copy_ceiling": head.get("copy_ceiling"),
        "cpu_baseline": head.get("cpu_baseline"),
        "kernels": results,
    }
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
