"""Roofline studies beside the benchmark (``python bench.py --hbm-ceiling |
--power | --data-energy | --vendor-gemm | --stage-table | --traffic-summary |
--mfma-summary``): HBM streaming ceilings from the bench-only probe library,
socket power, clock and throttle counters per step kernel, the vendor GEMM's
rate against K, per-stage Newton-Schulz rates, and summaries of rocprofv3
counter runs.  None of it is part of the optimizer step or of the benchmark
line; ``bench.py`` imports this module only for these flags.
"""
from __future__ import annotations

import ctypes as C
import json
import statistics
import time
from collections import defaultdict
from pathlib import Path

import torch

from bench import (PEAK_BF16_TFLOPS, PEAK_F32_TFLOPS, PEAK_HBM_GBS, ROOT, _ns_plan, build_gpu, kernel_symbol, log,
                   stage_exec_flops)


# ---------------------------------------------------------------- HBM ceiling
def probe_lib():
    """``bench_probe.so`` (built from ``bench_probe.hip`` by ``__graft_entry__.build()``):
    the HBM streaming probe, a library of its own apart from the optimizer's."""
    path = ROOT / "bench_probe.so"
    if not path.exists():
        raise RuntimeError(f"{path} is missing: build it with `python __graft_entry__.py`")
    lib = C.CDLL(str(path))
    lib.probe_hbm_stream.restype = C.c_int
    lib.probe_hbm_stream.argtypes = [C.c_int32, C.c_void_p, C.c_void_p, C.c_int64, C.c_int32, C.c_int32, C.c_void_p]
    lib.probe_last_error.restype = C.c_char_p
    return lib


def probe_check(lib, rc):
    if rc != 0:
        raise RuntimeError(f"probe_hbm_stream failed (code {rc}): {lib.probe_last_error().decode(errors='replace')}")


def hbm_ceiling(args):
    """Bandwidth of 16-B vector streams over 4 GiB buffers (probe_hbm_stream),
    swept over launch sizes and plain / non-temporal accesses, beside torch's
    device copy.  Two launch patterns: grid-stride 256-thread workgroups (4
    accesses in flight), and 1024-thread workgroups that each stream one
    contiguous span (8 in flight); with the spans also an in-place update
    (read and rewrite) and the momentum pack's three streams (gradient read,
    momentum read and rewritten, X written).  Bytes moved = read + written."""
    from monarch_muon_amd import _abi
    lib = probe_lib()
    dev = torch.device("cuda", 0)
    nbytes = 4 << 30
    gen = torch.Generator(device=dev).manual_seed(0)
    src = torch.randint(-2 ** 31, 2 ** 31 - 1, (nbytes // 4,), dtype=torch.int32, device=dev, generator=gen)
    dst = torch.empty_like(src)
    stream = _abi.stream_handle(dev)
    log(f"[bench] HBM ceiling on {torch.cuda.get_device_name(dev)}, {nbytes >> 30} GiB buffers")

    def timed(fn, reps=5):
        fn()
        torch.cuda.synchronize()
        ts = []
        for _ in range(reps):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            fn()
            b.record()
            b.synchronize()
            ts.append(a.elapsed_time(b))
        return statistics.median(ts)

    kinds = ((0, "read", "grid-stride", 1), (1, "write", "grid-stride", 1), (2, "copy", "grid-stride", 2),
             (3, "read", "spans", 1), (4, "write", "spans", 1), (5, "copy", "spans", 2),
             (6, "update in place", "spans", 2), (7, "pack pattern", "spans", 3))
    rows = []
    for kind, name, pattern, moved in kinds:
        grids = (1024, 2048, 4096, 8192, 16384) if pattern == "grid-stride" else (1024, 4096, 16384, 65536)
        for nt in (0, 1):
            for grid in grids:
                d = None if kind in (0, 3) else dst.data_ptr()
                ms = timed(lambda: probe_check(lib, lib.probe_hbm_stream(kind, d, src.data_ptr(), nbytes, nt, grid,
                                                                         stream)))
                rows.append({"kind": name, "pattern": pattern, "nontemporal": nt, "grid": grid, "ms": round(ms, 4),
                             "gbs": round(moved * nbytes / (ms * 1e-3) / 1e9, 1)})
    ms = timed(lambda: dst.copy_(src))
    rows.append({"kind": "copy", "pattern": "torch copy_", "nontemporal": None, "grid": None, "ms": round(ms, 4),
                 "gbs": round(2 * nbytes / (ms * 1e-3) / 1e9, 1)})
    best = {k: max((r for r in rows if r["kind"] == k), key=lambda r: r["gbs"])
            for k in ("read", "write", "copy", "update in place", "pack pattern")}
    print(json.dumps({"metric": "HBM stream bandwidth (GB/s, read + written)", "bytes": nbytes,
                      "peak_gbs": PEAK_HBM_GBS, "best": best, "rows": rows}), flush=True)


# ---------------------------------------------------------------- power and clock
class PowerSampler:
    """Socket power and GFX clock of this GPU (amdsmi), sampled from a thread
    every few ms, and the firmware's throttle accumulators."""

    def __init__(self, device):
        import amdsmi
        self.smi = amdsmi
        amdsmi.amdsmi_init()
        handles = amdsmi.amdsmi_get_processor_handles()
        if not handles:
            raise RuntimeError("amdsmi sees no GPU")
        self.h = handles[0]
        if len(handles) > 1:
            bus = torch.cuda.get_device_properties(device).pci_bus_id
            for h in handles:
                if int(amdsmi.amdsmi_get_gpu_device_bdf(h).split(":")[1], 16) == bus:
                    self.h = h
        self.samples = []
        self._stop = None

    VIOLATIONS = ("acc_counter", "acc_ppt_pwr", "acc_socket_thrm", "acc_vr_thrm", "acc_hbm_thrm", "acc_prochot_thrm")

    def violations(self):
        """Firmware throttle accumulators: acc_counter ticks, and the ticks during
        which each limiter held the clock (package power, socket / VR / HBM
        temperature, PROCHOT)."""
        try:
            v = self.smi.amdsmi_get_violation_status(self.h)
            return {k: v[k] for k in self.VIOLATIONS if isinstance(v.get(k), int)}
        except Exception:  # older firmware: no violation counters
            return {}

    def power_cap_w(self):
        try:
            return self.smi.amdsmi_get_power_cap_info(self.h)["power_cap"] / 1e6
        except Exception:
            return None

    def _read(self):
        m = self.smi.amdsmi_get_gpu_metrics_info(self.h)

        def num(x):
            return x if isinstance(x, (int, float)) else None

        clks = [c for c in (m.get("current_gfxclks") or []) if isinstance(c, (int, float)) and c > 0]
        clk = sum(clks) / len(clks) if clks else num(m.get("current_gfxclk"))
        return (time.perf_counter(), num(m.get("current_socket_power")), clk,
                num(m.get("average_gfxclk_frequency")), num(m.get("throttle_status")))

    def start(self):
        import threading
        self.samples = []
        self._stop = threading.Event()

        def loop():
            while not self._stop.is_set():
                try:
                    self.samples.append(self._read())
                except Exception:  # a failed read leaves a gap, nothing more
                    pass
                time.sleep(0.004)

        self._thread = threading.Thread(target=loop, daemon=True)
        self._thread.start()

    def stop(self, skip_s=0.3):
        self._stop.set()
        self._thread.join()
        t0 = self.samples[0][0] if self.samples else 0
        s = [x for x in self.samples if x[0] - t0 >= skip_s]

        def mean(i):
            v = [x[i] for x in s if x[i] is not None]
            return round(sum(v) / len(v), 1) if v else None
        return {"socket_w": mean(1), "gfx_mhz": mean(2), "avg_gfx_mhz": mean(3), "samples": len(s)}


def stage_bytes(kind, gl):
    """Algorithmic HBM bytes of one launch of a Newton-Schulz stage over the
    stored extents: bf16 X stacks (m_p x K rows x columns read, m_p x n_p
    written), the upper 256 x 256 tiles of A and P, and for the last PX the
    parameter block read and written instead of X'."""
    lay = gl.ws.layout
    N, mp, np_ = gl.nblocks, lay.mp, lay.np_
    if gl.struct.ns_dtype == 0:   # fp32 kernels: 128 x 128 tiles, SYRK / POLY the upper ones only
        kx = -(-lay.n // 32) * 32   # SYRK's K: n rounded up to the 32-deep K tiles
        nt = mp // 128
        up = (nt * (nt + 1) / 2) / (nt * nt)
        full = {"syrk": mp * mp * kx * up, "poly": mp ** 3 * up, "px": mp * mp * np_, "px_apply": mp * mp * np_}
        return 2.0 * full.get(kind, 0) * N
    nt = mp // 256
    up = nt * (nt + 1) // 2 * 256 * 256 * 2
    kx = -(-lay.n // 32) * 32
    xin = mp * kx * 2
    if kind == "syrk":
        return N * (xin + up)
    if kind == "poly":
        return N * 2 * up
    if kind == "symm":
        return N * 3 * up
    if kind == "px":
        return N * (up + xin + mp * np_ * 2)
    pb = 2 if gl.struct.param_dtype == 1 else 4
    return N * (up + xin + 2 * gl.rows * gl.cols * pb)


def stage_table(args, w):
    """Per group: each Newton-Schulz stage launched back to back (the second
    iteration's SYRK, POLY and PX, the last iteration's PX with the update),
    median over 3 loops of 20 launches, with its algorithmic HBM bytes and
    executed MFMA FLOPs per launch."""
    from monarch_muon_amd import _abi
    from monarch_muon_amd.optim import _COEFFS
    from monarch_muon_amd.plan import NS_STEPS
    dev = torch.device("cuda", 0)
    muon, adamw, opt = build_gpu(w, dev)
    opt.step()
    torch.cuda.synchronize()
    lib = _abi.lib()
    stream = _abi.stream_handle(dev)
    rows = []
    symm = _abi.NsOp(_abi.NSOP_SYMM, _abi.NSB_P, _abi.NSB_A, _abi.NSB_X1_S0, 0, 0)
    for gl in opt._muon_planner.groups:
        stages = [("syrk", 1, 0), ("poly", 1, 1), ("px", 1, 2), ("px_apply", NS_STEPS - 1, 2)]
        if any(op.kind == _abi.NSOP_SYMM for op in _ns_plan(gl, opt)):
            stages.insert(2, ("symm", 1, -1))
        for kind, it, st in stages:
            def launch():
                if st < 0:
                    _abi.check(lib.mmuon_ns_run_op(C.byref(gl.struct), C.byref(symm), _COEFFS, 0.0, stream),
                               "mmuon_ns_run_op")
                    return
                _abi.check(lib.mmuon_ns_stage(C.byref(gl.struct), it, NS_STEPS, st, _COEFFS,
                                              -0.02 * gl.alpha_scale, 0, stream), "mmuon_ns_stage")
            launch()
            torch.cuda.synchronize()
            loops = []
            for _ in range(3):
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                for _ in range(20):
                    launch()
                e1.record()
                torch.cuda.synchronize()
                loops.append(e0.elapsed_time(e1) / 20)
            ms = statistics.median(loops)
            nbytes = stage_bytes(kind, gl)
            ex = stage_exec_flops(kind, gl)
            rows.append({"group": f"{gl.rows}x{gl.cols}x{gl.nblocks}", "stage": kind, "ms": round(ms, 4),
                         "alg_bytes": nbytes, "gbs": round(nbytes / ms / 1e6, 1),
                         "frac_hbm": round(nbytes / ms / 1e6 / PEAK_HBM_GBS, 4),
                         "exec_tflops": round(ex / ms / 1e9, 1),
                         "frac_mfma": round(ex / ms / 1e9 / PEAK_BF16_TFLOPS, 4)})
            log(f"[stages] {rows[-1]}")
    print(json.dumps({"workload": w.name, "stages": rows}))


def vendor_gemm(args, w):
    """The vendor library's bf16 GEMM rate against the contraction length K
    (hipBLASLt through torch.mm, M = N = 8192, K = 1024 ... 8192; and the batched
    shape of the 1024 x 1024 group's PX), beside this build's PX launch of that
    group, all in one process: what a GEMM with PX's K = 1024 reaches on this GPU."""
    from monarch_muon_amd import _abi
    from monarch_muon_amd.optim import _COEFFS
    from monarch_muon_amd.plan import NS_STEPS
    dev = torch.device("cuda", 0)
    g = torch.Generator(device=dev).manual_seed(1)

    def timed(fn, reps=20):
        fn()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(reps):
            fn()
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b) / reps

    rows = []
    for k in (1024, 2048, 4096, 8192):
        A = torch.randn(8192, k, device=dev, generator=g).bfloat16()
        B = torch.randn(k, 8192, device=dev, generator=g).bfloat16()
        Out = torch.empty(8192, 8192, device=dev, dtype=torch.bfloat16)
        ms = timed(lambda: torch.mm(A, B, out=Out))
        rows.append({"case": f"torch.mm bf16 8192 x 8192 x {k} (hipBLASLt)", "k": k, "ms": round(ms, 4),
                     "tflops": round(2.0 * 8192 * 8192 * k / (ms * 1e-3) / 1e12, 1)})
        log(f"[vendor] {rows[-1]}")
        del A, B, Out
    A = torch.randn(1408, 1024, 1024, device=dev, generator=g).bfloat16()
    B = torch.randn(1408, 1024, 1024, device=dev, generator=g).bfloat16()
    Out = torch.empty_like(A)
    ms = timed(lambda: torch.bmm(A, B, out=Out))
    rows.append({"case": "torch.bmm bf16 1408 x 1024 x 1024 x 1024 (hipBLASLt, PX's shape)", "k": 1024,
                 "ms": round(ms, 4), "tflops": round(2.0 * 1408 * 1024 ** 3 / (ms * 1e-3) / 1e12, 1)})
    log(f"[vendor] {rows[-1]}")
    del A, B, Out
    muon, adamw, opt = build_gpu(w, dev)
    opt.step()
    torch.cuda.synchronize()
    lib = _abi.lib()
    gl = opt._muon_planner.groups[0]
    stream = _abi.stream_handle(dev)
    ms = timed(lambda: _abi.check(lib.mmuon_ns_stage(C.byref(gl.struct), 1, NS_STEPS, 2, _COEFFS, 0.0, 0, stream),
                                  "mmuon_ns_stage"))
    rows.append({"case": f"ns_px_bf16<2> PX, {gl.rows}x{gl.cols}x{gl.nblocks} group (this build)", "k": gl.rows,
                 "ms": round(ms, 4), "tflops": round(stage_exec_flops("px", gl) / (ms * 1e-3) / 1e12, 1)})
    log(f"[vendor] {rows[-1]}")
    print(json.dumps({"metric": "bf16 GEMM TFLOP/s against K", "rows": rows}), flush=True)


def power_rows(sampler, cases, flops, seconds, nbytes=None):
    """Each case launched back to back for about ``seconds``: ms per launch,
    sampled socket power and GFX clock, the limiters' share of the interval;
    executed TFLOP/s for the cases in ``flops``, GB/s for those in ``nbytes``.
    The first row is the idle GPU."""
    nbytes = nbytes or {}
    rows = []
    time.sleep(1.0)
    sampler.start()
    time.sleep(1.0)
    idle = sampler.stop(skip_s=0.2)
    rows.append({"kernel": "idle (nothing launched)", **idle})
    for name, fn in cases:
        fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        fn()
        torch.cuda.synchronize()
        one = time.perf_counter() - t0
        n = max(3, int(seconds / max(one, 1e-4)))
        sampler.start()
        time.sleep(0.05)
        v0 = sampler.violations()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(n):
            fn()
        b.record()
        torch.cuda.synchronize()
        v1 = sampler.violations()
        st = sampler.stop()
        ms = a.elapsed_time(b) / n
        row = {"kernel": name, "launches": n, "ms": round(ms, 4), **st}
        ticks = v1.get("acc_counter", 0) - v0.get("acc_counter", 0)
        if ticks > 0:
            row["limited_frac"] = {k[4:]: round((v1[k] - v0[k]) / ticks, 3) for k in v0
                                   if k != "acc_counter" and k in v1}
        if name in flops:
            row["exec_tflops"] = round(flops[name] / (ms * 1e-3) / 1e12, 1)
        if name in nbytes:
            row["gbs"] = round(nbytes[name] / (ms * 1e-3) / 1e9, 1)
        rows.append(row)
        log(f"[bench] {name}: {ms:.3f} ms, {st['socket_w']} W, {st['gfx_mhz']} MHz")
        time.sleep(0.5)
    return rows


def data_energy(args):
    """HBM power against the data moved: the same streams (read, and copy
    between two regions, 4 GiB each, 1024-thread workgroups streaming
    contiguous spans) over all-zero and over random-looking data, and the write
    probe's hashed data, each launched back to back under the power sampler."""
    from monarch_muon_amd import _abi
    lib = probe_lib()
    dev = torch.device("cuda", 0)
    nbytes = 4 << 30
    gen = torch.Generator(device=dev).manual_seed(0)
    rnd = torch.randint(-2 ** 31, 2 ** 31 - 1, (nbytes // 4,), dtype=torch.int32, device=dev, generator=gen)
    zero = torch.zeros_like(rnd)
    dst = torch.empty_like(rnd)
    stream = _abi.stream_handle(dev)
    sampler = PowerSampler(dev)

    def probe(kind, src, nt, out=None):
        return lambda: probe_check(lib, lib.probe_hbm_stream(kind, out, src.data_ptr(), nbytes, nt, 16384, stream))

    cases = [("read, all-zero data", probe(3, zero, 1)), ("read, random data", probe(3, rnd, 1)),
             ("copy, all-zero data", probe(5, zero, 1, dst.data_ptr())),
             ("copy, random data", probe(5, rnd, 1, dst.data_ptr())),
             ("write, hashed data", probe(4, rnd, 0, dst.data_ptr()))]
    moved = {"read, all-zero data": nbytes, "read, random data": nbytes, "copy, all-zero data": 2 * nbytes,
             "copy, random data": 2 * nbytes, "write, hashed data": nbytes}
    rows = power_rows(sampler, cases, {}, args.power_seconds, moved)
    print(json.dumps({"metric": "socket power / GFX clock against the data streamed", "bytes": nbytes,
                      "power_cap_w": sampler.power_cap_w(), "rows": rows}), flush=True)


def power_profile(args, w):
    """Each kernel of one optimizer step on the 1024 x 1024 group, the
    Gram-form stages of the shared rectangular unit, the AdamW group, the whole
    step and two vendor-library products, each launched back to back for about
    two seconds: ms per launch, socket power, GFX clock and the share of the
    interval the power limiter held the clock (power_rows)."""
    from monarch_muon_amd import _abi
    from monarch_muon_amd.optim import _COEFFS
    from monarch_muon_amd.plan import NS_STEPS
    dev = torch.device("cuda", 0)
    muon, adamw, opt = build_gpu(w, dev)
    opt.step()
    torch.cuda.synchronize()
    lib = _abi.lib()
    gl = opt._muon_planner.groups[0]
    stream = _abi.stream_handle(dev)
    sampler = PowerSampler(dev)
    alpha = -0.02 * gl.alpha_scale
    # the vendor library (hipBLASLt through torch) on the same batched shape as the
    # PX launch of this group, and on one large square product, under the same limits
    g = torch.Generator(device=dev).manual_seed(1)
    bm = min(gl.nblocks, 1408)
    A = torch.randn(bm, 1024, 1024, device=dev, generator=g).bfloat16()
    B = torch.randn(bm, 1024, 1024, device=dev, generator=g).bfloat16()
    Cb = torch.empty_like(A)
    X8 = torch.randn(8192, 8192, device=dev, generator=g).bfloat16()
    Y8 = torch.randn(8192, 8192, device=dev, generator=g).bfloat16()
    Z8 = torch.empty_like(X8)

    def stage(it, st):
        return lambda: _abi.check(lib.mmuon_ns_stage(C.byref(gl.struct), it, NS_STEPS, st, _COEFFS, alpha, 0, stream),
                                  "mmuon_ns_stage")

    cases = [
        ("pack_rows_kernel (1024x1024 group)",
         lambda: _abi.check(lib.mmuon_momentum_pack(C.byref(gl.struct), 0.95, stream), "pack")),
        ("ns_sym_bf16<0> SYRK (1024x1024 group, iteration 2)", stage(1, 0)),
        ("ns_sym_bf16<1> POLY (1024x1024 group, iteration 2)", stage(1, 1)),
        ("ns_px_bf16<2> PX (1024x1024 group, iteration 2)", stage(1, 2)),
        ("ns_px_bf16<3> PX + apply (1024x1024 group)", stage(NS_STEPS - 1, 2)),
        ("adamw_kernel (AdamW group)", lambda: opt._adamw_step(opt.param_groups[1], 0.02)),
        ("full optimizer step", lambda: opt.step()),
        (f"torch.bmm bf16 {bm} x 1024^3 (hipBLASLt, PX's shape)", lambda: torch.bmm(A, B, out=Cb)),
        ("torch.mm bf16 8192^3 (hipBLASLt)", lambda: torch.mm(X8, Y8, out=Z8)),
    ]
    flops = {cases[1][0]: stage_exec_flops("syrk", gl), cases[2][0]: stage_exec_flops("poly", gl),
             cases[3][0]: stage_exec_flops("px", gl), cases[4][0]: stage_exec_flops("px", gl),
             cases[7][0]: 2.0 * bm * 1024 ** 3, cases[8][0]: 2.0 * 8192 ** 3}
    # the Gram-form stages of the shared rectangular unit (2752 x 1024 + 1024 x 2752 blocks)
    from monarch_muon_amd.plan import BatchLaunch
    for u in opt._muon_planner.units:
        if not isinstance(u, BatchLaunch):
            continue
        name = "+".join(f"{m.rows}x{m.cols}" for m in u.members)
        ops = {o.kind: o for o in u.plan(NS_STEPS, opt._ns_flags)}
        sy = _abi.NsOp(_abi.NSOP_SYMM, _abi.NSB_P, _abi.NSB_A, _abi.NSB_X1_S0, 0, 0)
        for kind, op in (("syrk", ops.get(_abi.NSOP_SYRK)), ("poly", ops.get(_abi.NSOP_POLY)), ("symm", sy)):
            if op is None:
                continue
            label = f"{kernel_symbol(kind, u, 1)} {kind.upper()} ({name} unit, {u.nblocks} blocks)"
            cases.append((label, (lambda u=u, op=op: _abi.check(
                lib.mmuon_ns_run_op(C.byref(u.struct), C.byref(op), _COEFFS, 0.0, stream), "mmuon_ns_run_op"))))
            flops[label] = stage_exec_flops(kind, u)
    rows = power_rows(sampler, cases, flops, args.power_seconds)
    print(json.dumps({"metric": "socket power / GFX clock / energy per kernel", "workload": w.name,
                      "group": f"{gl.rows}x{gl.cols}x{gl.nblocks}", "power_cap_w": sampler.power_cap_w(),
                      "rows": rows}), flush=True)


# ---------------------------------------------------------------- rocprofv3 counter summaries
def short_kernel_name(name):
    """``void mmuon::(anonymous namespace)::ns_px_bf16<2, false, mmuon::(anonymous
    namespace)::BF16T>(mmuon::NsArgs, int)`` -> ``ns_px_bf16<2, false, BF16T>``."""
    n = name.strip().strip('"')
    if n.startswith("void "):
        n = n[5:]
    depth, cut = 0, len(n)
    for i, ch in enumerate(n):
        if ch == "<":
            depth += 1
        elif ch == ">":
            depth -= 1
        elif ch == "(" and depth == 0 and not n[i:].startswith("(anonymous"):
            cut = i
            break
    n = n[:cut]
    for pre in ("mmuon::(anonymous namespace)::", "mmuon::"):
        n = n.replace(pre, "")
    return n


def counter_summary(paths):
    """Per-kernel mean of every counter over the dispatches in rocprofv3
    ``*counter_collection.csv`` files, plus the mean dispatch duration (ns)."""
    import csv
    per = defaultdict(lambda: defaultdict(list))
    dur = defaultdict(dict)
    for path in paths:
        with open(path, newline="") as f:
            vals = defaultdict(float)
            for r in csv.DictReader(f):
                k = short_kernel_name(r["Kernel_Name"])
                key = (path, r["Dispatch_Id"], k)
                vals[key + (r["Counter_Name"],)] += float(r["Counter_Value"])
                if "Start_Timestamp" in r and r.get("End_Timestamp"):
                    dur[k][(path, r["Dispatch_Id"])] = int(r["End_Timestamp"]) - int(r["Start_Timestamp"])
        for (p_, d, k, c), v in vals.items():
            per[k][c].append(v)
    out = {}
    for k, cs in per.items():
        out[k] = {c: sum(v) / len(v) for c, v in cs.items()}
        out[k]["dispatches"] = max(len(v) for v in cs.values())
        if dur[k]:
            out[k]["duration_ns"] = sum(dur[k].values()) / len(dur[k])
    return out


def traffic_summary(args):
    """HBM bytes per dispatch from rocprofv3 counter runs of this script
    (``--traffic-summary OUT.json FETCH_CSV WRITE_CSV CAL_FETCH_CSV CAL_WRITE_CSV``):
    FETCH_SIZE and WRITE_SIZE (KiB) of every kernel, each scaled by what the same
    counter reads for ``--copy-calibration``'s 1 GiB copy; per kernel the mean
    over its dispatches, and for the Newton-Schulz and pack kernels of the last
    (instrumented) step of a 6.89B run, the value of every group and iteration
    (the instrumented step launches, per group in plan order, the pack, then
    SYRK, POLY, PX for each iteration)."""
    out_path, fetch_csv, write_csv, cal_f, cal_w = args.traffic_summary
    cf, cw = counter_summary([cal_f]), counter_summary([cal_w])
    copy = next(k for k in cf if "copyBuffer" in k or "copy" in k.lower())
    copy_bytes = 1 << 30
    fscale = copy_bytes / (cf[copy]["FETCH_SIZE"] * 1024)
    wscale = copy_bytes / (cw[copy]["WRITE_SIZE"] * 1024)
    f, wr = counter_summary([fetch_csv]), counter_summary([write_csv])
    kernels = {}
    for k in f:
        if k in wr and (k.startswith(("ns_", "pack", "adamw", "fp8_", "splitk")) or "butterfly" in k):
            b = f[k]["FETCH_SIZE"] * 1024 * fscale + wr[k]["WRITE_SIZE"] * 1024 * wscale
            kernels[k] = {"fetch_kib": f[k]["FETCH_SIZE"], "write_kib": wr[k]["WRITE_SIZE"], "bytes": b,
                          "read_bytes": f[k]["FETCH_SIZE"] * 1024 * fscale,
                          "write_bytes": wr[k]["WRITE_SIZE"] * 1024 * wscale, "dispatches": f[k]["dispatches"]}

    def seq(path, counter):
        import csv
        rows = {}
        with open(path, newline="") as fh:
            for r in csv.DictReader(fh):
                k = short_kernel_name(r["Kernel_Name"])
                if k.startswith(("ns_", "pack")) and r["Counter_Name"] == counter:
                    d = rows.setdefault(int(r["Dispatch_Id"]), [k, 0.0])
                    d[1] += float(r["Counter_Value"])
        return [rows[i] for i in sorted(rows)]

    fs, ws_ = seq(fetch_csv, "FETCH_SIZE"), seq(write_csv, "WRITE_SIZE")
    from monarch_muon_amd import _abi
    # the instrumented step's launches, unit by unit: the packs of the unit's
    # groups, the ops of its plan but the last over all its blocks, the last op
    # per group (the 6.89B units: the square group; the tall and wide groups)
    units = [[("1024x1024", 1408)], [("2752x1024", 256), ("1024x2752", 128)]]
    seq = []
    for members in units:
        n_all = sum(N for _, N in members)
        name = "+".join(g for g, _ in members)
        ops = _abi.ns_plan(1024, 1024 if members[0][0] == "1024x1024" else 2752, _abi.BF16, 5)
        seq += [None] * len(members)
        seq += [(name, n_all, op) for op in ops[:-1]]
        seq += [(g, N, ops[-1]) for g, N in members]
    per_group = []
    if len(fs) >= len(seq) and len(fs) == len(ws_):
        last_f, last_w = fs[-len(seq):], ws_[-len(seq):]
        for j, item in enumerate(seq):
            if item is None:
                continue
            name, N, op = item
            k, fk = last_f[j]
            per_group.append({"group": name, "iteration": op.iteration, "kernel": k,
                              "read_mib_per_block": round(fk * 1024 * fscale / N / 2 ** 20, 3),
                              "write_mib_per_block": round(last_w[j][1] * 1024 * wscale / N / 2 ** 20, 3)})
    Path(out_path).write_text(json.dumps({"calibration": {"fetch_scale": fscale, "write_scale": wscale},
                                          "kernels": kernels, "per_group": per_group}, indent=1) + "\n")
    print(json.dumps({k: round(v["bytes"] / 1e9, 3) for k, v in kernels.items()}, indent=1))


XCDS = 8  # MI355X: GRBM_GUI_ACTIVE is reported summed over the 8 XCDs' GRBMs


def mfma_summary(args):
    """MFMA utilisation per Newton-Schulz kernel, and the instruction mix of
    the streaming kernels, from rocprofv3 counter runs
    (``--mfma-summary OUT.json CSV...``): executed MFMA FLOP (SQ_INSTS_MFMA x
    32768, every instruction of the bf16 kernels being
    v_mfma_f32_32x32x16_bf16, x 4096 for the fp32 kernels' v_mfma_f32_32x32x2_f32;
    SQ_INSTS_VALU_MFMA_MOPS_BF16 / _F32 x 512 where collected), the
    GFX clock the counters imply (GRBM_GUI_ACTIVE / 8 XCDs / duration) and the
    MFMA busy fraction of all 1024 SIMDs' cycles (SQ_VALU_MFMA_BUSY_CYCLES /
    (GRBM_GUI_ACTIVE / 8 x 1024), rocprofv3's MfmaUtil).  For the pack, AdamW
    and FP8 kernels, where SQ_INSTS_VALU was collected: VALU, transcendental,
    vector-memory and LDS wave instructions per dispatch and their ratios."""
    out_path, *csvs = args.mfma_summary
    s = counter_summary(csvs)
    simds = 1024
    res = {}
    for k, c in s.items():
        if "duration_ns" not in c:
            continue
        secs = c["duration_ns"] * 1e-9
        rec = {"dispatches": c["dispatches"], "avg_ms": round(secs * 1e3, 4)}
        if k.startswith("ns_") and "SQ_INSTS_MFMA" in c:
            # bf16 kernels: v_mfma_f32_32x32x16_bf16 (32768 FLOP, 1024 FLOP per
            # SIMD cycle at peak); fp32 kernels: v_mfma_f32_32x32x2_f32 (4096
            # FLOP, 64 per SIMD cycle)
            f32 = k.startswith("ns_f32")
            flop = c["SQ_INSTS_MFMA"] * (4096.0 if f32 else 32768.0)
            peak = PEAK_F32_TFLOPS if f32 else PEAK_BF16_TFLOPS
            rec.update({"exec_flop": flop, "exec_tflops": round(flop / secs / 1e12, 1),
                        "exec_frac_peak": round(flop / secs / 1e12 / peak, 4)})
            if "SQ_INSTS_VALU_MFMA_MOPS_BF16" in c and not f32:
                rec["mops_flop"] = c["SQ_INSTS_VALU_MFMA_MOPS_BF16"] * 512.0
            if "SQ_INSTS_VALU_MFMA_MOPS_F32" in c and f32:
                rec["mops_flop"] = c["SQ_INSTS_VALU_MFMA_MOPS_F32"] * 512.0
            if "GRBM_GUI_ACTIVE" in c:
                cycles = c["GRBM_GUI_ACTIVE"] / XCDS
                rec["gfx_mhz"] = round(cycles / secs / 1e6, 1)
                # what the kernel executed against the peak at the clock it ran at
                rec["exec_frac_at_clock"] = round(flop / (cycles * simds * (64.0 if f32 else 1024.0)), 4)
                if "SQ_VALU_MFMA_BUSY_CYCLES" in c:
                    rec["mfma_busy"] = round(c["SQ_VALU_MFMA_BUSY_CYCLES"] / (cycles * simds), 4)
        elif k.startswith(("ns_", "pack", "adamw", "fp8_", "block_scale", "zero_pads")) and "SQ_INSTS_VALU" in c:
            # instruction mix (wave instructions summed over the device per dispatch)
            for name in ("SQ_INSTS_VALU", "SQ_INSTS_VALU_TRANS_F32", "SQ_INSTS_VMEM", "SQ_INSTS_LDS", "SQ_WAVES"):
                if name in c:
                    rec[name] = c[name]
            if c.get("SQ_INSTS_VMEM"):
                rec["valu_per_vmem"] = round(c["SQ_INSTS_VALU"] / c["SQ_INSTS_VMEM"], 2)
            if "SQ_INSTS_VALU_TRANS_F32" in c and c["SQ_INSTS_VALU"]:
                rec["trans_frac_of_valu"] = round(c["SQ_INSTS_VALU_TRANS_F32"] / c["SQ_INSTS_VALU"], 4)
            if "GRBM_GUI_ACTIVE" in c:
                cycles = c["GRBM_GUI_ACTIVE"] / XCDS
                rec["gfx_mhz"] = round(cycles / secs / 1e6, 1)
                # VALU wave instructions per SIMD cycle (a wave64 instruction
                # occupies its SIMD 4 cycles at full rate, 16 for a
                # quarter-rate transcendental)
                rec["valu_insts_per_simd_cycle"] = round(c["SQ_INSTS_VALU"] / (cycles * simds), 4)
        else:
            continue
        res[k] = rec
    Path(out_path).write_text(json.dumps({"simds": simds, "kernels": res}, indent=1) + "\n")
    print(json.dumps(res, indent=1))


def stall_summary(args):
    """Where each kernel's waves wait, from a rocprofv3 counter run
    (``--stall-summary OUT.json CSV``; counters SQ_WAVES, SQ_WAVE_CYCLES,
    SQ_WAIT_ANY, SQ_WAIT_INST_ANY, SQ_BUSY_CYCLES, SQ_LDS_BANK_CONFLICT,
    SQ_INSTS_LDS, SQ_INSTS_MFMA, GRBM_GUI_ACTIVE): per kernel the fraction of
    the waves' cycles spent waiting on a memory or LDS counter (SQ_WAIT_ANY /
    SQ_WAVE_CYCLES) and waiting to issue (SQ_WAIT_INST_ANY / SQ_WAVE_CYCLES,
    which includes a SIMD's other waves holding the issue slot), and LDS
    bank-conflict cycles per LDS instruction."""
    out_path, csv_path = args.stall_summary
    s = counter_summary([csv_path])
    res = {}
    for k, c in s.items():
        wc = c.get("SQ_WAVE_CYCLES", 0.0)
        if wc <= 0 or "duration_ns" not in c:
            continue
        if not (k.startswith(("ns_", "pack", "adamw", "fp8_", "splitk")) or "butterfly" in k):
            continue
        res[k] = {"dispatches": c["dispatches"], "avg_ms": round(c["duration_ns"] * 1e-6, 4),
                  "wait_any_frac": round(c["SQ_WAIT_ANY"] / wc, 3),
                  "wait_inst_frac": round(c["SQ_WAIT_INST_ANY"] / wc, 3),
                  "lds_conflict_cycles_per_lds_inst": round(c["SQ_LDS_BANK_CONFLICT"] / max(1.0, c["SQ_INSTS_LDS"]), 2)}
    Path(out_path).write_text(json.dumps({"kernels": res}, indent=1) + "\n")
    print(json.dumps(res, indent=1))
