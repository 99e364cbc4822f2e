"""Grouping and launch planner for the Monarch-Muon step.

The reference buckets the Muon parameters by ``(device, dtype, rows, cols)`` of
their momentum buffers, in first-appearance order, and concatenates each
bucket's blocks in parameter order (membench ``monarch_muon.py:153-161``).  The
planner reproduces that order exactly, but instead of copying the buffers into
a stack it builds a device table with one ``(param, grad, buf)`` pointer triple
per Monarch block; the fused pack kernel reads the blocks in place.  Tables and
workspaces are cached and rebuilt only when a pointer, dtype or shape changes.
"""
from __future__ import annotations

import ctypes as C
import math
from collections import OrderedDict
from dataclasses import dataclass, field

import numpy as np
import torch

from . import _abi

NS_COEFFS = (3.4445, -4.7750, 2.0315)   # membench monarch_muon.py:47
NS_STEPS = 5                            # membench monarch_muon.py:45


def group_key(buf: torch.Tensor):
    """``(device, dtype, rows, cols)`` of a momentum buffer (membench :156)."""
    return (buf.device, buf.dtype, buf.shape[1], buf.shape[2])


def plan_groups(bufs) -> "OrderedDict[tuple, list[int]]":
    """Indices of ``bufs`` per group key, keys in first-appearance order."""
    groups: "OrderedDict[tuple, list[int]]" = OrderedDict()
    for i, buf in enumerate(bufs):
        if buf.dim() != 3:
            raise ValueError(f"Muon parameters must be 3-D (nblocks, rows, cols); got shape {tuple(buf.shape)}")
        groups.setdefault(group_key(buf), []).append(i)
    return groups


def _h2d_int64(values, device) -> torch.Tensor:
    if isinstance(values, np.ndarray):
        host = torch.from_numpy(np.ascontiguousarray(values, dtype=np.int64)).pin_memory()
    else:
        host = torch.tensor(values, dtype=torch.int64).pin_memory()
    return host.to(device, non_blocking=True)


def _chunk_codes(numels, chunk: int) -> np.ndarray:
    """``tensor << 40 | first element`` of every ``chunk``-element chunk of the
    listed tensors, tensors in order (int64)."""
    n = np.asarray(numels, dtype=np.int64)
    per = (n + chunk - 1) // chunk
    total = int(per.sum())
    t = np.repeat(np.arange(n.size, dtype=np.int64), per)
    start = (np.arange(total, dtype=np.int64) - np.repeat(np.cumsum(per) - per, per)) * chunk
    return (t << 40) | start


class _KeyView:
    """A momentum buffer seen with another dtype for grouping (FP8 states are
    grouped by the dtype the wrapped reference step sees)."""

    def __init__(self, buf: torch.Tensor, dtype: torch.dtype):
        self.device, self.dtype, self.shape = buf.device, dtype, buf.shape

    def dim(self) -> int:
        return len(self.shape)


@dataclass
class Workspace:
    """Newton-Schulz workspace of one group geometry (owned by torch)."""
    layout: _abi.NsLayout
    x0: torch.Tensor
    x1: torch.Tensor
    a: torch.Tensor
    p: torch.Tensor
    partial: torch.Tensor
    scale: torch.Tensor

    @classmethod
    def allocate(cls, rows, cols, ns_code, nblocks, device, nparts: int = 0) -> "Workspace":
        """Stacks for ``nblocks`` blocks; ``nparts``: partial sums per block to
        make room for (at least the geometry's own)."""
        lay = _abi.ns_layout(rows, cols, ns_code, nblocks)
        u8 = dict(dtype=torch.uint8, device=device)
        part = nblocks * max(nparts, lay.nparts) * 4
        return cls(lay, torch.zeros(lay.x_bytes, **u8), torch.zeros(lay.x_bytes, **u8),
                   torch.empty(lay.a_bytes, **u8), torch.empty(lay.a_bytes, **u8),
                   torch.empty(max(part, 4), **u8),
                   torch.empty(nblocks, dtype=torch.float32, device=device))

    def view(self, lay: _abi.NsLayout, b0: int, nblocks: int, pstride: int) -> "Workspace":
        """Blocks ``b0 .. b0 + nblocks`` of these stacks as a workspace of their
        own with layout ``lay`` (same m, n, mp, np, dtype); ``pstride``: the
        partial sums reserved per block in this allocation."""
        xb = self.x0.numel() // self.scale.numel()   # bytes per block of each stack
        ab = self.a.numel() // self.scale.numel()
        pb = 4 * pstride
        return Workspace(lay, self.x0[b0 * xb:(b0 + nblocks) * xb], self.x1[b0 * xb:(b0 + nblocks) * xb],
                         self.a[b0 * ab:(b0 + nblocks) * ab], self.p[b0 * ab:(b0 + nblocks) * ab],
                         self.partial[b0 * pb:(b0 + nblocks) * pb], self.scale[b0:b0 + nblocks])

    def x_view(self, which: int, dtype: torch.dtype, nblocks: int) -> torch.Tensor:
        """The X stack (``which`` = 0 or 1) as ``[N, mp, np]``.  fp32 stacks are
        row-major (a view); bf16 stacks are stored in 32-column panels
        (``[N][np/32][mp][32]``) and come back as a row-major copy."""
        mp, np_ = self.layout.mp, self.layout.np_
        t = (self.x0 if which == 0 else self.x1).view(dtype)[:nblocks * mp * np_]
        if dtype == torch.float32:
            return t.view(nblocks, mp, np_)
        return t.view(nblocks, np_ // 32, mp, 32).permute(0, 2, 1, 3).reshape(nblocks, mp, np_)


@dataclass
class GroupLaunch:
    key: tuple
    rows: int
    cols: int
    nblocks: int
    members: list                 # indices into the step's param list, in order
    ws: Workspace
    table: torch.Tensor           # device int64 [N, 3]
    fp8_table: torch.Tensor | None
    struct: _abi.Group = field(default_factory=_abi.Group)
    # host copy of the table and what rebuilds its grad column alone
    rows_tab: np.ndarray | None = None    # int64 [N, 3]: param, grad, buf address of every block
    counts: np.ndarray | None = None      # blocks per member parameter
    kofs: np.ndarray | None = None        # block index within its parameter, per row
    grad_block_bytes: int = 0
    grad_dtype: torch.dtype | None = None
    ns_code: int = 0
    batch: "BatchLaunch | None" = None   # set when the group shares its Newton-Schulz launches

    @property
    def alpha_scale(self) -> float:
        return (self.rows / self.cols) ** 0.5   # membench :167

    @property
    def transposed(self) -> bool:
        return self.rows > self.cols


@dataclass
class BatchLaunch:
    """Groups of one Newton-Schulz geometry (device, NS dtype, m = min(r, c),
    n = max(r, c)) -- a tall group and its wide counterpart, e.g. 2752 x 1024
    and 1024 x 2752.  After the pack their blocks are all m x n stacks of the
    same layout, held in consecutive views of one workspace, so every
    Newton-Schulz launch but the last runs once over all of them; the last one
    (the apply) runs per group, with its parameters, orientation and
    ``sqrt(rows/cols)``.  Block results do not depend on the batch they run in,
    so this changes launches, not values."""
    members: list                 # GroupLaunch, in plan order
    ws: Workspace
    nblocks: int
    struct: _abi.Group = field(default_factory=_abi.Group)
    _plans: dict = field(default_factory=dict)

    def plan(self, iters: int, flags: int) -> list:
        """The ops ``mmuon_newton_schulz_apply`` would launch for these blocks."""
        k = (iters, flags)
        if k not in self._plans:
            self._plans[k] = _abi.ns_plan(self.rows, self.cols, self.struct.ns_dtype, iters, flags)
        return self._plans[k]

    @property
    def rows(self) -> int:
        return self.struct.rows

    @property
    def cols(self) -> int:
        return self.struct.cols

    @property
    def transposed(self) -> bool:
        return False

    def refresh(self) -> None:
        """Struct fields that follow the members' tables (rebuilt with new
        gradients).  The batch's launches never read the block table (only the
        apply does, and it runs per member); it points at the first member's."""
        s, first = self.struct, self.members[0].struct
        s.blocks = first.blocks
        s.flags = 0
        s.grad_scale = None


def ns_geometry(gl: "GroupLaunch"):
    """The key groups share Newton-Schulz launches under: (device, NS dtype, m, n)."""
    return (gl.key[0], gl.ns_code, min(gl.rows, gl.cols), max(gl.rows, gl.cols))


class MuonPlanner:
    """Builds and caches the per-step launch plan of the Muon group.

    The plan depends on the parameters, momentum buffers (and FP8 metadata)
    and on the gradients.  A training loop that drops its gradients after
    every step (``zero_grad(set_to_none=True)``) hands over new gradient
    tensors each step while everything else stays; then only the gradient
    column of each group's block table is recomputed and uploaded."""

    def __init__(self, merge: bool = True):
        self._sig = None
        self._gptr = None
        self._groups: list[GroupLaunch] = []
        self._units: list = []
        self._ws: dict = {}
        self._merge = merge

    @property
    def merge(self) -> bool:
        """Whether groups of one Newton-Schulz geometry share their launches
        (BatchLaunch); changing it rebuilds the plan at the next step."""
        return self._merge

    @merge.setter
    def merge(self, on: bool) -> None:
        if bool(on) != self._merge:
            self._merge = bool(on)
            self._sig = None

    @property
    def groups(self) -> list[GroupLaunch]:
        """The reference's groups, in its order (a group whose parameters differ
        in dtype appears as one entry per (param, grad) dtype pair, in order of
        first appearance)."""
        return self._groups

    @property
    def units(self) -> list:
        """Execution units in group order: a GroupLaunch, or a BatchLaunch for
        groups that share their Newton-Schulz launches (placed at its first
        member)."""
        return self._units

    def release(self) -> None:
        self._sig = None
        self._gptr = None
        self._groups = []
        self._units = []
        self._ws = {}

    def plan(self, params, grads, bufs, ns_dtype: torch.dtype, fp8_meta=None, key_dtypes=None) -> list[GroupLaunch]:
        """Launch plan of one step.  ``fp8_meta`` (FP8 states): per parameter,
        the (scale, expand, sqrt_minmax) tensors of an FP8 momentum buffer, or
        None where its buffer is a plain one.  ``key_dtypes`` (FP8 states): per parameter,
        the dtype the wrapped reference step sees for its momentum -- fp32 once
        dequantized, the parameter dtype when the buffer is created in this
        step -- used for the grouping key and, with ``ns_dtype=None``, as the
        Newton-Schulz dtype."""
        sig = tuple((p.data_ptr(), b.data_ptr(), p.dtype, b.dtype, b.shape) for p, b in zip(params, bufs))
        if fp8_meta is not None:
            sig = sig + tuple(t.data_ptr() if m is not None else None for m in fp8_meta for t in (m or (None,)))
        if key_dtypes is not None:
            sig = sig + tuple(key_dtypes)
        gptr = [(g.data_ptr(), g.dtype) for g in grads]
        if sig == self._sig:
            if gptr == self._gptr:
                return self._groups
            if self._regrad(params, grads, gptr):
                return self._groups
        keys = bufs if key_dtypes is None else [_KeyView(b, d) for b, d in zip(bufs, key_dtypes)]
        self._groups = []
        for key, idx in plan_groups(keys).items():
            # the reference keys a group on its buffers alone and applies per
            # parameter (membench :156, :165-170); parameters of one group whose
            # (param, grad) dtypes differ get a launch group each, which share
            # the group's Newton-Schulz launches (_link)
            subs: "OrderedDict[tuple, list[int]]" = OrderedDict()
            for i in idx:
                subs.setdefault((params[i].dtype, grads[i].dtype), []).append(i)
            self._groups += [self._build(key, sub, params, grads, bufs, ns_dtype, fp8_meta) for sub in subs.values()]
        self._link()
        self._sig, self._gptr = sig, gptr
        return self._groups

    def _regrad(self, params, grads, gptr) -> bool:
        """New gradient tensors, everything else unchanged: recompute and upload
        only the grad column of each table.  False (nothing changed) when a
        gradient's dtype, shape or layout differs from what its group was
        built for; the caller then rebuilds the plan, which validates."""
        for gl in self._groups:
            gd = gl.grad_dtype
            for i in gl.members:
                g = grads[i]
                if g.dtype != gd or g.shape != params[i].shape or not g.is_contiguous():
                    return False
        for gl in self._groups:
            gp = np.fromiter((gptr[i][0] for i in gl.members), dtype=np.int64, count=len(gl.members))
            rows_tab = gl.rows_tab.copy()
            rows_tab[:, 1] = np.repeat(gp, gl.counts) + gl.kofs * gl.grad_block_bytes
            gl.rows_tab = rows_tab
            # a new device table (the previous step's kernels may still read the old one)
            gl.table = _h2d_int64(rows_tab, gl.key[0])
            gl.struct.blocks = gl.table.data_ptr()
            gl.struct.flags = _abi.GROUP_ALIGNED16 if not bool(np.any(rows_tab % 16)) else 0
        for u in self._units:
            if isinstance(u, BatchLaunch):
                u.refresh()
        self._gptr = gptr
        return True

    def _workspace(self, m, n, ns_code, nblocks, device, pstride) -> Workspace:
        """One workspace per Newton-Schulz geometry (m <= n, NS dtype, device),
        grown to the largest batch seen; ``pstride`` partial sums per block."""
        k = (m, n, ns_code, device)
        ws = self._ws.get(k)
        if ws is None or ws.scale.numel() < nblocks or ws.partial.numel() < nblocks * pstride * 4:
            self._ws[k] = None  # drop the smaller one before allocating
            ws = self._ws[k] = Workspace.allocate(m, n, ns_code, nblocks, device, pstride)
        return ws

    def _link(self) -> None:
        """Give every group its workspace (consecutive views of one allocation
        per Newton-Schulz geometry) and form the execution units."""
        by_geo: "OrderedDict[tuple, list[GroupLaunch]]" = OrderedDict()
        for gl in self._groups:
            by_geo.setdefault(ns_geometry(gl) if self.merge else (id(gl),), []).append(gl)
        self._units = []
        for gls in by_geo.values():
            device, ns_code, m, n = ns_geometry(gls[0])
            lays = [_abi.ns_layout(gl.rows, gl.cols, ns_code, gl.nblocks) for gl in gls]
            pstride = max(lay.nparts for lay in lays)
            total = sum(gl.nblocks for gl in gls)
            ws = self._workspace(m, n, ns_code, total, device, pstride)
            b0 = 0
            for gl, lay in zip(gls, lays):
                gl.ws = ws.view(lay, b0, gl.nblocks, pstride)
                _point_at(gl.struct, gl.ws)
                gl.batch = None
                b0 += gl.nblocks
            if len(gls) == 1:
                self._units.append(gls[0])
                continue
            b = BatchLaunch(gls, ws.view(_abi.ns_layout(m, n, ns_code, total), 0, total, pstride), total)
            s, f = b.struct, gls[0].struct
            s.rows, s.cols, s.nblocks = m, n, total
            s.param_dtype, s.grad_dtype, s.buf_dtype, s.ns_dtype = f.param_dtype, f.grad_dtype, f.buf_dtype, ns_code
            s.fp8 = None
            _point_at(s, b.ws)
            b.refresh()
            for gl in gls:
                gl.batch = b
            self._units.append(b)

    def _build(self, key, idx, params, grads, bufs, ns_dtype, fp8_meta) -> GroupLaunch:
        device, kdtype, rows, cols = key
        bdtype = bufs[idx[0]].dtype
        rc = rows * cols
        pd, gd = params[idx[0]].dtype, grads[idx[0]].dtype
        for i in idx:
            p, g, b = params[i], grads[i], bufs[i]
            if p.dtype != pd or g.dtype != gd:
                raise TypeError("a launch group's parameters (and their grads) must share a dtype")
            if not (p.is_contiguous() and g.is_contiguous() and b.is_contiguous()):
                raise ValueError("Muon parameters, grads and momentum buffers must be contiguous")
            if p.shape != b.shape or g.shape != p.shape:
                raise ValueError("param, grad and momentum shapes differ")
        if ns_dtype is not None:
            ns_code = _abi.dtype_code(ns_dtype)
        elif kdtype in _abi.FP8_DTYPES:
            ns_code = _abi.F32          # the FP8 reference dequantizes the momentum to fp32
        else:
            ns_code = _abi.dtype_code(kdtype)
        counts = np.array([bufs[i].shape[0] for i in idx], dtype=np.int64)
        nblocks = int(counts.sum())
        es = np.array([params[idx[0]].element_size(), grads[idx[0]].element_size(),
                       bufs[idx[0]].element_size()], dtype=np.int64) * rc
        bases = np.array([(params[i].data_ptr(), grads[i].data_ptr(), bufs[i].data_ptr()) for i in idx],
                         dtype=np.int64)
        k = np.arange(nblocks, dtype=np.int64) - np.repeat(np.cumsum(counts) - counts, counts)
        rows_tab = np.repeat(bases, counts, axis=0) + k[:, None] * es[None, :]
        aligned = not bool(np.any(rows_tab % 16))
        table = _h2d_int64(rows_tab, device)
        fp8_table = None
        if fp8_meta is not None and bdtype in _abi.FP8_DTYPES:
            if any(fp8_meta[i] is None for i in idx):
                raise ValueError("FP8 momentum buffers need their metadata")
            mb = np.array([tuple(t.data_ptr() for t in fp8_meta[i]) for i in idx], dtype=np.int64)
            fp8_table = _h2d_int64(np.repeat(mb, counts, axis=0) + k[:, None] * (rc // 128 * 4), device)
        gl = GroupLaunch(key, rows, cols, nblocks, list(idx), None, table, fp8_table, rows_tab=rows_tab,
                         counts=counts, kofs=k, grad_block_bytes=int(es[1]), grad_dtype=gd, ns_code=ns_code)
        s = gl.struct
        s.rows, s.cols, s.nblocks = rows, cols, nblocks
        s.param_dtype, s.grad_dtype = _abi.dtype_code(pd), _abi.dtype_code(gd)
        s.buf_dtype = _abi.dtype_code(bdtype)
        s.ns_dtype = ns_code
        s.flags = _abi.GROUP_ALIGNED16 if aligned else 0
        s.blocks = table.data_ptr()
        s.fp8 = fp8_table.data_ptr() if fp8_table is not None else None
        return gl   # workspace pointers: _link


def _point_at(s: _abi.Group, ws: Workspace) -> None:
    s.x0, s.x1 = ws.x0.data_ptr(), ws.x1.data_ptr()
    s.a, s.p = ws.a.data_ptr(), ws.p.data_ptr()
    s.partial, s.scale = ws.partial.data_ptr(), ws.scale.data_ptr()


def run_newton_schulz(units, lib, coeffs, lr: float, flags: int, iters: int, stream_of, pack) -> None:
    """One step's Muon launches, unit by unit: the pack of every group (``pack(gl,
    stream)``), then Newton-Schulz and the apply -- ``mmuon_newton_schulz_apply``
    for a lone group; for a batch, the same call with ``NS_HOLD_LAST`` over all
    member blocks (every op of the plan but the last), then the last op (the
    apply) per member with its own alpha."""
    for u in units:
        if isinstance(u, BatchLaunch):
            stream = stream_of(u.members[0])
            for gl in u.members:
                pack(gl, stream)
            ops = u.plan(iters, flags)
            _abi.check(lib.mmuon_newton_schulz_apply(C.byref(u.struct), iters, coeffs, 0.0,
                                                     flags | _abi.NS_HOLD_LAST, stream), "mmuon_newton_schulz_apply")
            for gl in u.members:
                _abi.check(lib.mmuon_ns_run_op(C.byref(gl.struct), C.byref(ops[-1]), coeffs,
                                               -lr * gl.alpha_scale, stream), "mmuon_ns_run_op")
        else:
            stream = stream_of(u)
            pack(u, stream)
            _abi.check(lib.mmuon_newton_schulz_apply(C.byref(u.struct), iters, coeffs, -lr * u.alpha_scale,
                                                     flags, stream), "mmuon_newton_schulz_apply")


# ---------------------------------------------------------------------------
# AdamW group
# ---------------------------------------------------------------------------
ADAM_CHUNK = 8192


@dataclass
class AdamLaunch:
    members: list                 # indices into the step's param list
    pd: torch.dtype
    gd: torch.dtype
    sd: torch.dtype               # exp_avg dtype
    tensors: torch.Tensor         # device int64 [T, 5]
    chunks: torch.Tensor          # device int64 [nchunks]
    nchunks: int
    chunk: int
    fp8: torch.Tensor | None = None  # device int64 [T, 6]
    host: np.ndarray | None = None   # host copy of `tensors`
    vd: torch.dtype | None = None    # exp_avg_sq dtype (differs from sd only for FP8 states)


class AdamPlanner:
    """Device tables of the AdamW launch; when only the gradients are new
    tensors, only their column of the tensor table is rewritten."""

    def __init__(self):
        self._sig = None
        self._gptr = None
        self._launches: list[AdamLaunch] = []

    def release(self) -> None:
        self._sig = None
        self._gptr = None
        self._launches = []

    def plan(self, params, grads, ms, vs, fp8_meta=None) -> list[AdamLaunch]:
        sig = tuple((p.data_ptr(), m.data_ptr(), v.data_ptr(), p.dtype, m.dtype, v.dtype, p.numel())
                    for p, m, v in zip(params, ms, vs))
        if fp8_meta is not None:
            sig = sig + tuple(t.data_ptr() for meta in fp8_meta for t in meta)
        gptr = [(g.data_ptr(), g.dtype) for g in grads]
        if sig == self._sig:
            if gptr == self._gptr:
                return self._launches
            if self._regrad(params, grads, gptr):
                return self._launches
        buckets: "OrderedDict[tuple, list[int]]" = OrderedDict()
        for i, (p, g, m, v) in enumerate(zip(params, grads, ms, vs)):
            if m.dtype != v.dtype and fp8_meta is None:
                raise TypeError("exp_avg and exp_avg_sq must share a dtype")
            for t in (p, g, m, v):
                if not t.is_contiguous():
                    raise ValueError("AdamW parameters, grads and states must be contiguous")
            buckets.setdefault((p.device, p.dtype, g.dtype, m.dtype, v.dtype), []).append(i)
        launches = []
        chunk = 128 if fp8_meta is not None else ADAM_CHUNK
        for (device, pd, gd, sd, vd), idx in buckets.items():
            tens = np.array([(params[i].data_ptr(), grads[i].data_ptr(), ms[i].data_ptr(), vs[i].data_ptr(),
                              params[i].numel()) for i in idx], dtype=np.int64).reshape(-1, 5)
            chunks = _chunk_codes([params[i].numel() for i in idx], chunk)
            f8 = [tuple(x.data_ptr() for x in fp8_meta[i]) for i in idx] if fp8_meta is not None else None
            launches.append(AdamLaunch(
                idx, pd, gd, sd, _h2d_int64(tens, device), _h2d_int64(chunks if chunks.size else [0], device),
                int(chunks.size), chunk, _h2d_int64(f8, device) if f8 is not None else None, host=tens, vd=vd))
        self._launches = launches
        self._sig, self._gptr = sig, gptr
        return launches

    def _regrad(self, params, grads, gptr) -> bool:
        """New gradient tensors only: rewrite their column of each tensor table.
        False when a gradient's dtype, size or layout differs from its bucket's
        (the caller then rebuilds, which validates)."""
        for al in self._launches:
            for i in al.members:
                g = grads[i]
                if g.dtype != al.gd or g.numel() != params[i].numel() or not g.is_contiguous():
                    return False
        for al in self._launches:
            host = al.host.copy()
            host[:, 1] = np.fromiter((gptr[i][0] for i in al.members), dtype=np.int64, count=len(al.members))
            al.host = host
            al.tensors = _h2d_int64(host, al.tensors.device)  # the previous launch may still read the old one
        self._gptr = gptr
        return True


def adamw_scalars(lr, beta1, beta2, eps, weight_decay, step) -> dict:
    """Scalars exactly as the reference forms them in Python doubles
    (membench monarch_muon.py:196-208)."""
    bc1 = 1.0 - beta1 ** step
    bc2 = 1.0 - beta2 ** step
    return dict(apply_weight_decay=int(weight_decay > 0), wd_factor=1.0 - lr * weight_decay,
                beta1=beta1, beta2=beta2, one_minus_beta1=1.0 - beta1, one_minus_beta2=1.0 - beta2,
                sqrt_bc2=math.sqrt(bc2), eps=eps, neg_step_size=-lr / bc1)


# ---------------------------------------------------------------------------
# Gradient-norm clipping (the norm pass of torch.nn.utils.clip_grad_norm_)
# ---------------------------------------------------------------------------
NORM_CHUNK = 8192


@dataclass
class NormLaunch:
    dtype: torch.dtype
    tensors: torch.Tensor         # device int64 [T, 2]: gradient pointer, numel
    chunks: torch.Tensor          # device int64 [nchunks]: tensor << 40 | first element
    first_chunk: torch.Tensor     # device int64 [T + 1]
    nchunks: int
    ntensors: int
    partial: torch.Tensor         # fp32 [nchunks] workspace
    norms: torch.Tensor           # fp32 [T] workspace
    total: torch.Tensor           # fp32 [1]
    coef: torch.Tensor            # fp32 [1]


class NormPlanner:
    """Device tables for the gradient-norm pass; rebuilt only when a gradient
    pointer, dtype or size changes."""

    def __init__(self):
        self._sig = None
        self._launch: NormLaunch | None = None

    def release(self) -> None:
        self._sig = None
        self._launch = None

    def plan(self, grads) -> NormLaunch:
        sig = tuple((g.data_ptr(), g.dtype, g.numel(), g.device) for g in grads)
        if sig == self._sig:
            return self._launch
        if len({g.dtype for g in grads}) != 1 or len({g.device for g in grads}) != 1:
            raise NotImplementedError("fused gradient clipping needs every gradient on one device in one dtype")
        for g in grads:
            if not g.is_contiguous():
                raise ValueError("gradients must be contiguous")
        device = grads[0].device
        numels = [g.numel() for g in grads]
        tens = [(g.data_ptr(), n) for g, n in zip(grads, numels)]
        chunks = _chunk_codes(numels, NORM_CHUNK)
        per = (np.asarray(numels, dtype=np.int64) + NORM_CHUNK - 1) // NORM_CHUNK
        first = np.concatenate([[0], np.cumsum(per)]).astype(np.int64)
        f32 = dict(dtype=torch.float32, device=device)
        self._launch = NormLaunch(grads[0].dtype, _h2d_int64(tens, device),
                                  _h2d_int64(chunks if chunks.size else [0], device),
                                  _h2d_int64(first, device), int(chunks.size), len(grads),
                                  torch.empty(max(1, int(chunks.size)), **f32), torch.empty(max(1, len(grads)), **f32),
                                  torch.empty(1, **f32), torch.empty(1, **f32))
        self._sig = sig
        return self._launch
