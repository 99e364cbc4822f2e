"""Monarch-Muon optimizer-step benchmark on one MI355X.

    python bench.py [--steps K] [--warmup W] [--workload 6.89b-nb4] [--no-cpu-baseline]
    python bench.py --workload butterfly-6.89b [--tokens 4096]
    python bench.py --hbm-ceiling          # read / write / copy bandwidth of this GPU (bench_studies.py)
    python bench.py --power                # socket power and GFX clock per step kernel (bench_studies.py)

Runs the full ``MonarchMuonOptimizer.step()`` (Muon group: momentum, bf16
Newton-Schulz over every Monarch block, apply; AdamW group) of the named
workload on synthetic data already resident in HBM, times exactly K steps
between two device synchronisations, and prints one JSON line.  The dominant
kernel's roofline comes from per-launch hipEvents on the launch stream over
extra instrumented steps; the CPU baseline times the oracle (the CPU
restatement of the reference step) on a bounded sample of the same workload.

After the timed steps, a second leg replaces every gradient with a freshly
allocated tensor before each step, as ``zero_grad(set_to_none=True)`` and the
next backward do in the reference's training loop, and reports the host time
the launch planners spend rebuilding their pointer tables (``host_plan_ms``).

``--workload butterfly-<model>`` times the Monarch butterfly multiply instead:
forward + backward of one transformer layer's seven Monarch projections
(q, k, v, o, gate, up, down) at ``--tokens`` rows (default 4096, the reference
benchmark's micro-batch 4 x sequence 1024), beside the reference's own torch
ops for the same layer run on the same GPU.
"""
from __future__ import annotations

import argparse
import ctypes as C
import gc
import json
import os
import statistics
import sys
import time
from collections import defaultdict
from pathlib import Path

import torch

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "optimizer-step ms, 6.89B-ref nb=4 bf16; NS TFLOP/s as % of bf16 MFMA peak"
PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
PEAK_F32_TFLOPS = 157.3     # MI355X dense fp32 MFMA
PEAK_HBM_GBS = 8000.0
REFERENCE_H100_MS = 304.4   # README.md:16 (bf16 momentum, H100)


def log(*a):
    print(*a, file=sys.stderr, flush=True)


# ---------------------------------------------------------------- workload
def build_gpu(w, device, seed=0, ns_form="auto", merge=True):
    from monarch_muon_amd import CoatStateMonarchMuon, MonarchMuonOptimizer, QuantizationConfig, _abi
    from monarch_muon_amd.workloads import parameter_inventory
    gen = torch.Generator(device=device).manual_seed(seed)
    muon, adamw, bufs = [], [], []
    for _, shape, is_muon in parameter_inventory(w):
        p = (torch.randn(shape, generator=gen, device=device) * 0.02).to(w.param_dtype).requires_grad_(True)
        p.grad = (torch.randn(shape, generator=gen, device=device) * 1e-3).to(w.param_dtype)
        (muon if is_muon else adamw).append(p)
        if is_muon and w.prefill_momentum:
            bufs.append(torch.randn(shape, generator=gen, device=device) * 1e-3)
    if w.momentum_dtype == "fp8":
        opt = CoatStateMonarchMuon(muon, adamw, lr=0.02, momentum=0.95, qargs=QuantizationConfig(),
                                   ns_dtype=w.ns_dtype, ns_form=ns_form)
        for p, b in zip(muon, bufs):
            st = opt.state[p]
            groups = (b.numel() + 127) // 128
            codes = torch.empty(b.shape, dtype=torch.float8_e4m3fn, device=device)
            meta = [torch.empty(groups, dtype=torch.float32, device=device) for _ in range(3)]
            _abi.fp8_quantize(b.contiguous(), codes.view(torch.uint8), *meta, signed=True)
            st["momentum_buffer"] = codes
            for key, t in zip(("scale", "expand", "sqrt_minmax"), meta):
                st[f"{key}_momentum_buffer"] = t
    else:
        opt = MonarchMuonOptimizer(muon, adamw, lr=0.02, momentum=0.95, ns_dtype=w.ns_dtype, ns_form=ns_form)
        for p, b in zip(muon, bufs):
            opt.state[p]["momentum_buffer"] = b.to(w.momentum_dtype)
    del bufs
    opt._muon_planner.merge = merge
    torch.cuda.synchronize()
    return muon, adamw, opt


# ---------------------------------------------------------------- per-kernel timing
def instrumented_step(opt, lr=0.02):
    """One optimizer step with a hipEvent pair around every launch (on the
    stream the kernels run on).  Returns [(kernel, group, seconds_event_pair)]."""
    from monarch_muon_amd import _abi
    from monarch_muon_amd.optim import _COEFFS
    from monarch_muon_amd.plan import NS_STEPS, BatchLaunch
    lib = _abi.lib()
    out = []
    muon_group, adam_group = opt.param_groups
    fp8 = type(opt).__name__ == "CoatStateMonarchMuon"

    def timed(kind, gl, it, fn):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        fn()
        e1.record()
        out.append((kind, gl, it, e0, e1))

    def pack(gl, stream):
        if fp8:
            _abi.check(lib.mmuon_fp8_momentum_pack(C.byref(gl.struct), 0.95, 1, float(opt.expand_min), stream),
                       "pack")
        else:
            _abi.check(lib.mmuon_momentum_pack(C.byref(gl.struct), 0.95, stream), "pack")

    def run_op(unit, op, alpha, stream):
        _abi.check(lib.mmuon_ns_run_op(C.byref(unit.struct), C.byref(op), _COEFFS, alpha, stream),
                   "mmuon_ns_run_op")

    # the launches of a step, one at a time, unit by unit (plan.run_newton_schulz)
    for u in opt._muon_planner.units:
        members = u.members if isinstance(u, BatchLaunch) else [u]
        stream = _abi.stream_handle(members[0].key[0])
        for gl in members:
            timed("pack", gl, 0, lambda: pack(gl, stream))
        ops = _abi.ns_plan(u.rows, u.cols, u.struct.ns_dtype, NS_STEPS, opt._ns_flags)
        for op in ops[:-1]:
            timed(OP_KIND[op.kind], u, op.iteration, lambda: run_op(u, op, 0.0, stream))
        for gl in members:
            timed(OP_KIND[ops[-1].kind], gl, ops[-1].iteration,
                  lambda: run_op(gl, ops[-1], -lr * gl.alpha_scale, stream))
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    opt._adamw_step(adam_group, lr)
    e1.record()
    out.append(("adamw", None, 0, e0, e1))
    torch.cuda.synchronize()
    return [(k, gl, it, e0.elapsed_time(e1)) for k, gl, it, e0, e1 in out]


# Newton-Schulz plan op kinds (MMUON_NSOP_*) by name
OP_KIND = {0: "syrk", 1: "poly", 2: "px", 3: "px_apply", 4: "symm"}
NS_KINDS = ("syrk", "poly", "symm", "px", "px_apply")


def kernel_symbol(kind, gl, it, fp8=False):
    """The kernel (template instance) rocprof reports for a launch, as it
    appears in ``rocprofv3 --stats`` names (mmuon::(anonymous namespace)::...)."""
    tp = "BF16T" if gl is not None and gl.struct.param_dtype == 1 else "F32T"
    if gl is not None and kind in NS_KINDS and gl.struct.ns_dtype == 0:  # fp32 Newton-Schulz
        stage = {"syrk": 0, "poly": 1, "px": 2, "px_apply": 3}[kind]
        return f"ns_f32<{stage}, {tp if stage == 3 else 'F32T'}>"
    if kind == "syrk":
        return "ns_sym_bf16<0>"
    if kind == "poly":
        return "ns_sym_bf16<1>"
    if kind == "symm":
        return "ns_sym_bf16<4>"
    if kind == "px":
        return "ns_px_bf16<2, false, BF16T>"
    if kind == "px_apply":
        return f"ns_px_bf16<3, {'true' if gl.transposed else 'false'}, {tp}>"
    if kind == "pack":
        return ("fp8_" if fp8 else "") + ("pack_cols_kernel" if gl.transposed else "pack_rows_kernel")
    return kind + ("_fp8_kernel" if fp8 else "_kernel")


def stage_flops(kind, gl):
    """Algorithmic FLOPs of one launch (its full product, symmetry not credited)."""
    lay = gl.ws.layout
    m, n, N = lay.m, lay.n, gl.nblocks
    if kind == "syrk":
        return 2.0 * m * m * n * N
    if kind in ("poly", "symm"):
        return 2.0 * m * m * m * N
    if kind in ("px", "px_apply"):
        return 2.0 * m * m * n * N
    return 0.0


def stage_exec_flops(kind, gl):
    """MFMA FLOPs the kernels execute (padded tiles; symmetric stages compute the
    256x256 tiles above the diagonal, and on a diagonal tile the 36 of its 64
    32x32 MFMA tiles on or above the diagonal)."""
    lay = gl.ws.layout
    N, mp, np_ = gl.nblocks, lay.mp, lay.np_
    if gl.struct.ns_dtype == 0:   # fp32 kernels: 128 x 128 tiles, SYRK / POLY the upper ones only
        kx = -(-lay.n // 32) * 32   # SYRK's K: n rounded up to the 32-deep K tiles
        nt = mp // 128
        up = (nt * (nt + 1) / 2) / (nt * nt)
        full = {"syrk": mp * mp * kx * up, "poly": mp ** 3 * up, "px": mp * mp * np_, "px_apply": mp * mp * np_}
        return 2.0 * full.get(kind, 0) * N
    nt = mp // 256
    sym = (nt * (nt - 1) / 2 + nt * 36 / 64) / (nt * nt)
    kx = -(-lay.n // 32) * 32   # SYRK's K: n rounded up to the 32-deep slices
    if kind == "syrk":
        return 2.0 * mp * mp * kx * N * sym
    if kind in ("poly", "symm"):
        return 2.0 * mp * mp * mp * N * sym
    if kind in ("px", "px_apply"):
        return 2.0 * mp * mp * np_ * N
    return 0.0


def _ns_plan(gl, opt):
    from monarch_muon_amd import _abi
    from monarch_muon_amd.plan import NS_STEPS
    return _abi.ns_plan(gl.rows, gl.cols, gl.struct.ns_dtype, NS_STEPS, opt._ns_flags)


def pack_bytes(gl, momentum_bytes, grad_bytes=2, x_bytes=2):
    lay = gl.ws.layout
    return gl.nblocks * lay.m * lay.n * (grad_bytes + 2 * momentum_bytes + x_bytes)


def adamw_bytes(w):
    """Algorithmic AdamW bytes: param read + write, grad read, both moments read
    + write (1-byte codes on the FP8 path, metadata not counted)."""
    from monarch_muon_amd.workloads import adamw_elements
    pb = torch.empty((), dtype=w.param_dtype).element_size()
    sb = 1 if w.momentum_dtype == "fp8" else pb
    return adamw_elements(w) * (3 * pb + 4 * sb)


def hbm_traffic(workload, kernel):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 counter
    summary (FETCH_SIZE and WRITE_SIZE, each scaled by a plain copy's reading);
    None when no summary covers this workload and kernel."""
    path = ROOT / "profiles" / f"hbm_traffic_{workload}.json"
    try:
        data = json.loads(path.read_text())
        return round(data["kernels"][kernel]["bytes"])
    except (OSError, KeyError, ValueError):
        return None


# ---------------------------------------------------------------- CPU baseline
CPU_SAMPLE_LAYERS = 4


def freeze_gc():
    """Collect, then move every object alive now (torch's ~170K import-time
    objects, the workload) into the collector's permanent generation, so a full
    collection -- 50-70 ms of host time -- cannot land inside a timed region
    while the GPU queue is still short (it showed as one ~125 ms step right after
    the warm-up).  The collector stays enabled for new objects.  Called before
    the warm-up, so the timed steps follow the warm-up without an idle gap."""
    gc.collect()
    gc.freeze()


def host_cpu_info(threads):
    """What the CPU baseline ran on: model string, logical CPUs this process
    may use, the physical cores behind them, and the threads used."""
    model, cores = "", set()
    cur, first = {}, {}
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if not line.strip():
                    if "processor" in cur:
                        cores.add((int(cur["processor"]), cur.get("physical id", "0"), cur.get("core id", cur["processor"])))
                        first = first or cur
                    cur = {}
                    continue
                k, _, v = line.partition(":")
                cur[k.strip()] = v.strip()
                if k.strip() == "model name" and not model:
                    model = v.strip()
            if "processor" in cur:
                cores.add((int(cur["processor"]), cur.get("physical id", "0"), cur.get("core id", cur["processor"])))
    except OSError:
        pass
    allowed = sorted(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else list(range(os.cpu_count() or 1))
    phys = {(pid, cid) for proc, pid, cid in cores if proc in allowed}
    flags = set(first.get("flags", "").split())
    names = {"vendor_id": "cpu_vendor", "cpu family": "cpu_family", "model": "cpu_model_number",
             "stepping": "cpu_stepping", "cpu MHz": "cpu_mhz"}
    ident = {v: first[k] for k, v in names.items() if k in first}
    return {"cpu_model": model, **ident, "hypervisor": "hypervisor" in flags,
            "avx512_bf16": "avx512_bf16" in flags, "threads": threads, "logical_cpus_allowed": len(allowed),
            "physical_cores_allowed": len(phys) or None, "os_cpu_count": os.cpu_count()}


def cpu_baseline(w, seed=0):
    """The oracle step on the host cores over a bounded sample: the Muon blocks
    of the first CPU_SAMPLE_LAYERS transformer layers plus the same fraction of
    the AdamW elements; scaled to one full step."""
    from oracle.step import ReferenceMonarchMuon
    from monarch_muon_amd.workloads import local_layers, parameter_inventory
    allowed = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    threads = max(1, min(16, allowed))
    torch.set_num_threads(threads)
    nl = local_layers(w)
    layers = min(CPU_SAMPLE_LAYERS, nl)
    gen = torch.Generator().manual_seed(seed)
    muon, adamw, bufs = [], [], []
    for name, shape, is_muon in parameter_inventory(w):
        if ".h." in name and int(name.split(".")[2]) >= layers:
            continue
        if not is_muon and (len(shape) == 2 or w.shards > 1):
            shape = (max(1, shape[0] * layers // nl), *shape[1:])
        p = (torch.randn(shape, generator=gen) * 0.02).to(w.param_dtype).requires_grad_(True)
        p.grad = (torch.randn(shape, generator=gen) * 1e-3).to(w.param_dtype)
        (muon if is_muon else adamw).append(p)
        if is_muon:
            bufs.append(torch.randn(shape, generator=gen) * 1e-3)
    variant = "membench" if w.ns_dtype == torch.bfloat16 else "pretrain"
    opt = ReferenceMonarchMuon(muon, adamw, lr=0.02, momentum=0.95, variant=variant)
    for p, b in zip(muon, bufs):
        opt.state[p]["momentum_buffer"] = b if w.momentum_dtype == "fp8" else b.to(w.momentum_dtype)
    opt.step()  # warm-up
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        opt.step()
        times.append(time.perf_counter() - t0)
    sample_ms = statistics.median(times) * 1e3
    scale = nl / layers
    return {"value": round(sample_ms * scale, 1), "unit": "ms", "cores": threads, "kind": "port",
            "sample": f"oracle step (torch CPU) over the Muon blocks of layers 0-{layers - 1} + {layers}/{nl} "
                      f"of the AdamW elements, median of 3 after 1 warm-up = {sample_ms:.1f} ms, x{scale:g}",
            **host_cpu_info(threads)}


# ---------------------------------------------------------------- butterfly
BUTTERFLY_METRIC = "Monarch layer fwd+bwd ms (7 butterfly projections), bf16; TFLOP/s as % of bf16 MFMA peak"


def butterfly_layer(w, tokens, device, seed=0):
    """The seven Monarch projections of one layer: [(name, x, w1, w2, dout)], bf16."""
    from monarch_muon_amd.workloads import factor_shapes, mlp_hidden
    hid = mlp_hidden(w.n_embd, w.intermediate)
    dims = [("q", w.n_embd, w.n_embd), ("k", w.n_embd, w.n_embd), ("v", w.n_embd, w.n_embd),
            ("o", w.n_embd, w.n_embd), ("gate", w.n_embd, hid), ("up", w.n_embd, hid), ("down", hid, w.n_embd)]
    g = torch.Generator(device=device).manual_seed(seed)
    out = []
    for name, d_in, d_out in dims:
        s1, s2 = factor_shapes(d_in, d_out, w.nblocks)
        x = torch.randn(tokens, s1[0] * s1[2], device=device, generator=g).bfloat16()
        w1 = (torch.randn(*s1, device=device, generator=g) / s1[2] ** 0.5).bfloat16()
        w2 = (torch.randn(*s2, device=device, generator=g) / s2[2] ** 0.5).bfloat16()
        dout = torch.randn(tokens, s2[0], s2[1], device=device, generator=g).bfloat16()
        out.append((name, x, w1, w2, dout))
    return out


def butterfly_flops(x, w1, w2):
    """Forward flops of one projection (two batched products); the backward is twice this."""
    k, q, p = w1.shape
    l, s, r = w2.shape
    return 2 * x.shape[0] * (k * q * p + l * s * r)


def torch_reference_fwd(x2, w1, w2):
    """pretrain/src/models/monarch/monarch_ops.py:23-36 with the eager riffle (right operands made
    contiguous: transposed bf16 bmm operands are avoided on this platform)."""
    B = x2.shape[0]
    k, q, p = w1.shape
    l, s, r = w2.shape
    out1 = torch.bmm(x2.reshape(B, k, p).transpose(0, 1), w1.transpose(-1, -2).contiguous())
    t = out1.transpose(0, 1).reshape(B, r, l).permute(2, 0, 1).contiguous()
    return torch.bmm(t, w2.transpose(-1, -2).contiguous()).transpose(0, 1).contiguous(), t


def torch_reference_bwd(x2, w1, w2, out1, dout_blk):
    """monarch_ops.py:57-82 with the eager unriffle."""
    B = x2.shape[0]
    k, q, p = w1.shape
    l, s, r = w2.shape
    d = dout_blk.permute(1, 0, 2)
    dw2 = torch.bmm(d.transpose(-1, -2).contiguous(), out1)
    dt = torch.bmm(d.contiguous(), w2)
    dout1 = dt.transpose(0, 1).transpose(-1, -2).contiguous().reshape(B, k, q).transpose(0, 1).contiguous()
    dx = torch.bmm(dout1, w1).transpose(0, 1).reshape(B, k * p)
    dw1 = torch.bmm(dout1.transpose(-1, -2).contiguous(), x2.reshape(B, k, p).transpose(0, 1).contiguous())
    return dx, dw1, dw2


def butterfly_cpu_baseline(layer):
    """The oracle (torch CPU) forward + backward of every projection of the layer at 1/8 of the
    tokens, scaled by 8."""
    from oracle import butterfly as bf
    allowed = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    threads = max(1, min(16, allowed))
    torch.set_num_threads(threads)
    frac = 8
    cpu = [(x[: x.shape[0] // frac].cpu(), w1.cpu(), w2.cpu(), d[: d.shape[0] // frac].cpu())
           for _, x, w1, w2, d in layer]

    def run():
        for x, w1, w2, d in cpu:
            _, o1 = bf.butterfly_fwd(x, w1, w2)
            bf.butterfly_bwd(x, w1, w2, o1, d)

    run()
    t0 = time.perf_counter()
    run()
    sample_ms = (time.perf_counter() - t0) * 1e3
    return {"value": round(sample_ms * frac, 1), "unit": "ms", "cores": threads, "kind": "port",
            "sample": f"oracle butterfly fwd+bwd (torch CPU, fp32 products of bf16 values) of the 7 projections "
                      f"at {cpu[0][0].shape[0]} tokens = {sample_ms:.1f} ms after 1 warm-up, x{frac}",
            **host_cpu_info(threads)}


def bench_butterfly(args, w):
    from monarch_muon_amd import butterfly_blk_bwd_op, butterfly_blk_op
    dev = torch.device("cuda", 0)
    tokens = args.tokens
    log(f"[bench] butterfly layer of {w.name}, {tokens} tokens, on {torch.cuda.get_device_name(dev)}")
    layer = butterfly_layer(w, tokens, dev)
    fwd_fl = sum(butterfly_flops(x, w1, w2) for _, x, w1, w2, _ in layer)
    saved = {}

    def step():
        for name, x, w1, w2, _ in layer:
            saved[name] = butterfly_blk_op(x, w1, w2)[1]
        for name, x, w1, w2, d in reversed(layer):
            butterfly_blk_bwd_op(x, w1, w2, saved[name], d)

    freeze_gc()
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
    t0 = time.perf_counter()
    for a, b in evs:
        a.record()
        step()
        b.record()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / args.steps
    ev_ms = statistics.median(a.elapsed_time(b) for a, b in evs)

    # per-op times (hipEvents on the launch stream, which is torch's current stream)
    def op_ms(fn, reps=10):
        fn()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        a.record()
        for _ in range(reps):
            fn()
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b) / reps

    per = {}
    fwd_ms = bwd_ms = ref_fwd_ms = ref_bwd_ms = 0.0
    for name, x, w1, w2, d in layer:
        fl = butterfly_flops(x, w1, w2)
        f = op_ms(lambda: butterfly_blk_op(x, w1, w2))
        o1 = butterfly_blk_op(x, w1, w2)[1]
        bw = op_ms(lambda: butterfly_blk_bwd_op(x, w1, w2, o1, d))
        rf = op_ms(lambda: torch_reference_fwd(x, w1, w2))
        rt = torch_reference_fwd(x, w1, w2)[1]
        rb = op_ms(lambda: torch_reference_bwd(x, w1, w2, rt, d))
        fwd_ms, bwd_ms, ref_fwd_ms, ref_bwd_ms = fwd_ms + f, bwd_ms + bw, ref_fwd_ms + rf, ref_bwd_ms + rb
        per[name] = {"w1": list(w1.shape), "w2": list(w2.shape), "fwd_ms": round(f, 4), "bwd_ms": round(bw, 4),
                     "fwd_tflops": round(fl / (f * 1e-3) / 1e12, 1), "bwd_tflops": round(2 * fl / (bw * 1e-3) / 1e12, 1),
                     "torch_fwd_ms": round(rf, 4), "torch_bwd_ms": round(rb, 4)}
    # the dominant kernel: the forward product (two launches of butterfly_gemm<false, false, false>
    # per forward call; the event pair around the call also holds the gap between them)
    fwd_avg_launch = fwd_ms / (2 * len(layer))
    achieved = fwd_fl / (fwd_ms * 1e-3) / 1e12
    total_fl = 3 * fwd_fl
    res = {
        "metric": BUTTERFLY_METRIC, "value": round(wall_ms, 4), "unit": "ms", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(wall_ms, 4), "higher_is_better": False, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) activations and gradients, N(0,1/fan_in) factors, resident in HBM)",
        "config": {"workload": f"butterfly-{w.name.split('-')[0]}", "tokens": tokens, "nblocks": w.nblocks,
                   "hidden": w.n_embd, "intermediate": w.intermediate, "projections": 7,
                   "step": "forward of the 7 projections, then their backward in reverse order"},
        "median_event_ms": round(ev_ms, 4),
        "tflops": round(total_fl / (wall_ms * 1e-3) / 1e12, 1),
        "frac_peak": round(total_fl / (wall_ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
        "roofline": {"bound": "mfma", "kernel": "butterfly_gemm<false, false, false>", "achieved": round(achieved, 1),
                     "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s", "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
                     "traffic": hbm_traffic("butterfly-6.89b" if tokens == 4096 and w.name == "6.89b-nb4" else "-",
                                            "butterfly_gemm<false, false, false>"),
                     "avg_launch_ms": round(fwd_avg_launch, 4),
                     "alg_flops_per_launch": fwd_fl / (2 * len(layer))},
        "forward_ms": round(fwd_ms, 4), "backward_ms": round(bwd_ms, 4),
        "torch_reference_ms": {"forward": round(ref_fwd_ms, 4), "backward": round(ref_bwd_ms, 4),
                               "total": round(ref_fwd_ms + ref_bwd_ms, 4),
                               "note": "the reference's monarch_ops.py bmm + eager riffle path, same GPU, per-op events"},
        "projections": per,
    }
    if not args.no_cpu_baseline:
        log("[bench] CPU baseline (oracle on host cores, bounded sample)")
        res["cpu_baseline"] = butterfly_cpu_baseline(layer)
    print(json.dumps(res), flush=True)


# ---------------------------------------------------------------- fresh gradients
def fresh_grad_leg(opt, params, steps=5):
    """Steps whose every gradient is a newly allocated tensor at a new address
    (the previous step's gradients are still held while the new ones are
    allocated), as in a training loop that drops the gradients after each step
    (``zero_grad(set_to_none=True)``, pretrain/src/optim/base.py:125) and gets
    new ones from the next backward.  The planners then rebuild their pointer
    tables every step.  Returns host ms spent in the planners, host ms of the
    whole ``step()`` call, and wall ms per step (synchronised)."""
    saved = [p.grad for p in params]
    spent = [0.0]
    planners = (opt._muon_planner, opt._adam_planner)

    def timed(fn):
        def wrapper(*a, **k):
            t0 = time.perf_counter()
            try:
                return fn(*a, **k)
            finally:
                spent[0] += time.perf_counter() - t0
        return wrapper

    for pl in planners:
        pl.plan = timed(pl.plan)   # instance attribute shadows the method
    plan_ms, host_ms, wall_ms = [], [], []
    try:
        for i in range(steps + 1):
            fresh = [g.clone() for g in saved]
            for p, g in zip(params, fresh):
                p.grad = g
            del fresh
            torch.cuda.synchronize()
            spent[0] = 0.0
            t0 = time.perf_counter()
            opt.step()
            t1 = time.perf_counter()
            torch.cuda.synchronize()
            t2 = time.perf_counter()
            if i:  # the leg's first step is dropped like a warm-up
                plan_ms.append(spent[0] * 1e3)
                host_ms.append((t1 - t0) * 1e3)
                wall_ms.append((t2 - t0) * 1e3)
    finally:
        for pl in planners:
            del pl.plan
        for p, g in zip(params, saved):
            p.grad = g
    return {"host_plan_ms": round(statistics.median(plan_ms), 3),
            "host_step_call_ms": round(statistics.median(host_ms), 3),
            "step_ms": round(statistics.median(wall_ms), 3), "steps": steps,
            "note": "every gradient reallocated at a new address before each step; planners rebuild their tables"}


def mfma_util(workload, kernel):
    """The committed MFMA-counter summary of `kernel` at `workload`, or None."""
    try:
        data = json.loads((ROOT / "profiles" / f"mfma_util_{workload}.json").read_text())
        return data["kernels"][kernel]
    except (OSError, KeyError, ValueError):
        return None


# ---------------------------------------------------------------- main
def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=12)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default="6.89b-nb4")
    ap.add_argument("--tokens", type=int, default=4096, help="butterfly workloads: rows of the layer input")
    ap.add_argument("--instrumented", type=int, default=2, help="extra per-kernel-timed steps")
    ap.add_argument("--separate-groups", action="store_true",
                    help="launch every group's Newton-Schulz on its own (by default a tall group and its wide "
                         "counterpart share their launches)")
    ap.add_argument("--ns-form", choices=("auto", "standard"), default="auto",
                    help="Newton-Schulz evaluation order (the optimizer's ns_form): auto = the Gram form for "
                         "the rectangular bf16 groups, standard = the three-product chain everywhere")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--grad-clip", type=float, default=0.0,
                    help="also clip the gradient norm before every timed step (opt.clip_grad_norm_), and report "
                         "the fused clip and torch.nn.utils.clip_grad_norm_ on the same gradients")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a plain 1 GiB device-to-device copy (for HBM counter calibration)")
    ap.add_argument("--fresh-steps", type=int, default=5,
                    help="steps of the fresh-gradient leg (host planner time); 0 skips it")
    ap.add_argument("--hbm-ceiling", action="store_true", help="only measure read / write / copy bandwidth")
    ap.add_argument("--power", action="store_true",
                    help="only measure socket power, GFX clock and the power limiter per step kernel")
    ap.add_argument("--power-seconds", type=float, default=2.0)
    ap.add_argument("--data-energy", action="store_true",
                    help="only measure socket power and clock while streaming all-zero against random data")
    ap.add_argument("--vendor-gemm", action="store_true",
                    help="only measure hipBLASLt's bf16 GEMM rate against K beside this build's PX launch")
    ap.add_argument("--stage-table", action="store_true",
                    help="time each Newton-Schulz stage per group: ms, algorithmic GB/s, executed TFLOP/s")
    ap.add_argument("--traffic-summary", nargs=5,
                    metavar=("OUT_JSON", "FETCH_CSV", "WRITE_CSV", "CAL_FETCH_CSV", "CAL_WRITE_CSV"),
                    help="summarise rocprofv3 FETCH_SIZE / WRITE_SIZE runs into OUT_JSON (HBM bytes per dispatch)")
    ap.add_argument("--mfma-summary", nargs="+", metavar=("OUT_JSON", "CSV"),
                    help="summarise rocprofv3 counter CSVs (SQ_INSTS_MFMA, SQ_VALU_MFMA_BUSY_CYCLES, "
                         "GRBM_GUI_ACTIVE; or SQ_INSTS_VALU, SQ_INSTS_VALU_TRANS_F32, SQ_INSTS_VMEM, "
                         "SQ_INSTS_LDS) into OUT_JSON")
    ap.add_argument("--stall-summary", nargs=2, metavar=("OUT_JSON", "CSV"),
                    help="summarise a rocprofv3 counter CSV (SQ_WAVE_CYCLES, SQ_WAIT_ANY, SQ_WAIT_INST_ANY, "
                         "SQ_LDS_BANK_CONFLICT, SQ_INSTS_LDS) into OUT_JSON: where each kernel's waves wait")
    args = ap.parse_args()
    if args.stall_summary:
        import bench_studies
        bench_studies.stall_summary(args)
        return
    if args.mfma_summary:
        import bench_studies
        bench_studies.mfma_summary(args)
        return
    if args.traffic_summary:
        import bench_studies
        bench_studies.traffic_summary(args)
        return
    if args.copy_calibration:
        x = torch.ones(2 ** 28, dtype=torch.float32, device="cuda")
        y = torch.empty_like(x)
        y.copy_(x)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes_read": x.numel() * 4, "copy_bytes_written": y.numel() * 4}))
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures the single-GPU optimizer step only; multi-GPU runs are not part of "
              "this build (a sharded step would give each GPU its own share of the Newton-Schulz blocks).",
              file=sys.stderr)
        sys.exit(2)
    from monarch_muon_amd.workloads import WORKLOADS, adamw_elements, local_layers, muon_elements, ns_flops
    if args.hbm_ceiling or args.power or args.vendor_gemm or args.data_energy or args.stage_table:
        import bench_studies
        if args.hbm_ceiling:
            bench_studies.hbm_ceiling(args)
        elif args.power:
            bench_studies.power_profile(args, WORKLOADS[args.workload])
        elif args.vendor_gemm:
            bench_studies.vendor_gemm(args, WORKLOADS[args.workload])
        elif args.data_energy:
            bench_studies.data_energy(args)
        else:
            bench_studies.stage_table(args, WORKLOADS[args.workload])
        return
    if args.workload.startswith("butterfly-"):
        model = args.workload[len("butterfly-"):]
        base = next(k for k in WORKLOADS if k.split("-")[0] == model)
        bench_butterfly(args, WORKLOADS[base])
        return
    w = WORKLOADS[args.workload]
    dev = torch.device("cuda", 0)
    log(f"[bench] building workload {w.name} on {torch.cuda.get_device_name(dev)}")
    muon, adamw, opt = build_gpu(w, dev, ns_form=args.ns_form, merge=not args.separate_groups)
    freeze_gc()
    log(f"[bench] warm-up {args.warmup} steps")
    for _ in range(args.warmup):
        if args.grad_clip:
            opt.clip_grad_norm_(args.grad_clip)
        opt.step()
    torch.cuda.synchronize()
    log(f"[bench] timing {args.steps} steps")
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for s, e in evs:
        s.record()
        if args.grad_clip:
            opt.clip_grad_norm_(args.grad_clip)
        opt.step()
        e.record()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / args.steps
    step_ms = [s.elapsed_time(e) for s, e in evs]
    median_ms = statistics.median(step_ms)
    log(f"[bench] {wall_ms:.2f} ms/step (wall), median event {median_ms:.2f} ms; per-step events (ms): "
        + " ".join(f"{v:.1f}" for v in step_ms))

    # per-kernel timing
    per = defaultdict(lambda: [0.0, 0, 0.0, 0.0])   # symbol -> [ms, launches, alg flops, exec flops]
    stage_ms = defaultdict(float)
    for _ in range(max(1, args.instrumented)):
        for kind, gl, it, ms in instrumented_step(opt):
            sym = kernel_symbol(kind, gl, it, fp8=w.momentum_dtype == "fp8")
            rec = per[sym]
            rec[0] += ms
            rec[1] += 1
            if gl is not None:
                rec[2] += stage_flops(kind, gl)
                rec[3] += stage_exec_flops(kind, gl)
            stage_ms[kind] += ms
    reps = max(1, args.instrumented)
    ns_ms = sum(stage_ms[k] for k in NS_KINDS) / reps
    ns_tf = ns_flops(w) / (ns_ms * 1e-3) / 1e12
    ns_exec = sum(v[3] for k, v in per.items() if k.startswith("ns_")) / reps
    dominant = max((k for k in per if k.startswith("ns_")), key=lambda k: per[k][0])
    d_ms, d_n, d_fl, d_ex = per[dominant]
    d_avg = d_ms / d_n
    achieved = (d_fl / d_n) / (d_avg * 1e-3) / 1e12
    traffic = hbm_traffic(w.name, dominant)
    counters = mfma_util(w.name, dominant)
    kernels = {k: {"avg_ms": round(v[0] / v[1], 4), "launches_per_step": v[1] // reps,
                   "ms_per_step": round(v[0] / reps, 3),
                   **({"alg_tflops": round(v[2] / (v[0] * 1e-3) / 1e12, 1),
                       "exec_tflops": round(v[3] / (v[0] * 1e-3) / 1e12, 1)} if v[2] else {})}
               for k, v in sorted(per.items(), key=lambda kv: -kv[1][0])}
    mom_bytes = 4 if w.momentum_dtype == torch.float32 else (2 if w.momentum_dtype == torch.bfloat16 else 1)
    pack_ms = stage_ms["pack"] / reps
    gbytes = torch.empty((), dtype=w.param_dtype).element_size()
    pack_b = sum(pack_bytes(gl, mom_bytes, gbytes, 4 if gl.struct.ns_dtype == 0 else 2)
                 for gl in opt._muon_planner.groups)
    # Newton-Schulz in fp32 (the pretrain copy with fp32 momentum): priced against the fp32 MFMA peak
    ns32 = w.ns_dtype is None and w.momentum_dtype in (torch.float32, "fp8")
    peak = PEAK_F32_TFLOPS if ns32 else PEAK_BF16_TFLOPS
    res = {
        "metric": METRIC, "value": round(wall_ms, 3), "unit": "ms", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(wall_ms, 3), "higher_is_better": False,
        "scaling": "weak", "vs_baseline": None, "dtype": "fp32" if ns32 else "bf16",
        "data": "synthetic (seeded N(0,.02) weights, N(0,1e-3) grads and momentum, resident in HBM)",
        "config": {"workload": w.name, "layers": w.n_layer, "hidden": w.n_embd, "intermediate": w.intermediate,
                   **({"shard": f"rank 0 of {w.shards}: the Muon blocks of layers 0-{local_layers(w) - 1} and 1/{w.shards} "
                                f"of the AdamW group's elements"} if w.shards > 1 else {}),
                   "nblocks": w.nblocks, "muon_elements": muon_elements(w), "adamw_elements": adamw_elements(w),
                   "param_dtype": str(w.param_dtype).split(".")[-1],
                   "momentum_dtype": w.momentum_dtype if isinstance(w.momentum_dtype, str)
                   else str(w.momentum_dtype).split(".")[-1],
                   "newton_schulz": ("fp32 MFMA" if ns32 else "bf16 MFMA, fp32 accumulate") + ", 5 iterations",
                   "ns_form": args.ns_form, "shared_launches": not args.separate_groups,
                   "groups": [f"{gl.rows}x{gl.cols}x{gl.nblocks}" for gl in opt._muon_planner.groups]},
        "median_event_ms": round(median_ms, 3),
        "event_ms": {"min": round(min(step_ms), 3), "mean": round(statistics.mean(step_ms), 3),
                     "median": round(median_ms, 3), "max": round(max(step_ms), 3)},
        "statistics": {"value": "wall-clock mean of the K timed steps between two device synchronisations "
                                "(the Python collector's existing objects frozen before timing)",
                       "median_event_ms": "median of per-step hipEvent pairs, the reference harness's statistic "
                                          "(benchmark_train_step.py:297-299,386-397: 3 warm-ups, median of 12 "
                                          "event-timed steps; this script's defaults)"},
        "roofline": {"bound": "mfma", "kernel": dominant, "achieved": round(achieved, 1),
                     "peak": peak, "unit": "TFLOP/s", "frac": round(achieved / peak, 4),
                     "traffic": traffic, "avg_launch_ms": round(d_avg, 4),
                     "alg_flops_per_launch": d_fl / d_n, "exec_tflops": round((d_ex / d_n) / (d_avg * 1e-3) / 1e12, 1),
                     **({"exec_frac": round((d_ex / d_n) / (d_avg * 1e-3) / 1e12 / peak, 4),
                         "counters": {"source": f"profiles/mfma_util_{w.name}.json",
                                      **{k: counters[k] for k in ("exec_frac_peak", "exec_frac_at_clock",
                                                                  "mfma_busy", "gfx_mhz") if k in counters}}}
                        if counters else {})},
        "newton_schulz": {"ms": round(ns_ms, 3), "alg_tflop": round(ns_flops(w) / 1e12, 2),
                          "alg_tflops": round(ns_tf, 1), "chain_equiv_frac_peak": round(ns_tf / peak, 4),
                          "exec_tflop": round(ns_exec / 1e12, 2),
                          "exec_tflops": round(ns_exec / (ns_ms * 1e-3) / 1e12, 1),
                          "exec_frac_peak": round(ns_exec / (ns_ms * 1e-3) / 1e12 / peak, 4),
                          "peak_tflops": peak,
                          "forms": {f"{gl.rows}x{gl.cols}x{gl.nblocks}":
                                    "gram" if any(op.kind == 4 for op in _ns_plan(gl, opt)) else "chain"
                                    for gl in opt._muon_planner.groups},
                          "note": "alg_tflop: the reference's three-product chain (2m^2(2n+m) per block and "
                                  "iteration, symmetric products counted in full), the work every evaluation "
                                  "order replaces; exec_tflop: the MFMA work the launched kernels execute; "
                                  "chain_equiv_frac_peak: the chain's work per second over the peak, not MFMA "
                                  "utilisation (exec_frac_peak is)"},
        "momentum_pack": {"ms": round(pack_ms, 3), "alg_bytes": pack_b,
                          "gbs": round(pack_b / (pack_ms * 1e-3) / 1e9, 1),
                          "frac_hbm": round(pack_b / (pack_ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)},
        "muon_group_ms": round(sum(stage_ms[k] for k in ("pack",) + NS_KINDS) / reps, 3),
        "adamw_ms": round(stage_ms["adamw"] / reps, 3),
        "adamw_gbs": round(adamw_bytes(w) / (stage_ms["adamw"] / reps * 1e-3) / 1e9, 1),
        "kernels": kernels,
        "reference_h100_ms": REFERENCE_H100_MS,
    }
    if w.momentum_dtype == torch.bfloat16 and w.name.startswith("6.89b"):
        # the states the published H100 step time was measured with (bf16 params, grads, momentum)
        res["vs_baseline"] = round(wall_ms / REFERENCE_H100_MS, 4)
        res["vs_baseline_note"] = "value / 304.4 ms (README.md:16, 1x H100, bf16 momentum); lower is faster"
    if args.grad_clip:
        params = muon + adamw

        def timed(fn, reps=5):
            fn()
            torch.cuda.synchronize()
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            for _ in range(reps):
                fn()
            b.record()
            torch.cuda.synchronize()
            return a.elapsed_time(b) / reps

        fused = timed(lambda: opt.clip_grad_norm_(args.grad_clip))
        ref = timed(lambda: torch.nn.utils.clip_grad_norm_(params, args.grad_clip))  # rescales the grads in place
        res["grad_clip"] = {"max_norm": args.grad_clip, "fused_clip_ms": round(fused, 3),
                            "torch_clip_grad_norm_ms": round(ref, 3),
                            "note": "value/ms_per_step include opt.clip_grad_norm_ before every step"}
    if args.fresh_steps > 0:
        log(f"[bench] fresh-gradient leg ({args.fresh_steps} steps)")
        res["fresh_grads"] = fresh_grad_leg(opt, muon + adamw, args.fresh_steps)
        res["host_plan_ms"] = res["fresh_grads"]["host_plan_ms"]
    if not args.no_cpu_baseline:
        log("[bench] CPU baseline (oracle on host cores, bounded sample)")
        res["cpu_baseline"] = cpu_baseline(w)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
