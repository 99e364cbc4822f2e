"""Drop-in ``MonarchMuonOptimizer`` and ``CoatStateMonarchMuon`` on MI355X kernels.

Same constructor, param groups, ``step``/``state_dict`` behaviour and state
keys as the reference (``membench/src/models/monarch/monarch_muon.py:57-208``,
``pretrain/src/models/monarch/monarch_muon.py:57-201``,
``pretrain/src/models/monarch/coat_state_muon.py:117-151``).  Every step runs
on the GPU through ``libmmuon.so``; parameters must live on a ROCm device.

``ns_dtype`` selects which reference copy is reproduced:
``torch.bfloat16`` (default) -- the membench copy: each same-shape stack is
cast to bf16 for Newton-Schulz (the published-step-time variant);
``None`` -- the pretrain copy: Newton-Schulz in the momentum dtype.

``ns_form`` selects how bf16 Newton-Schulz is evaluated for rectangular groups:
``"auto"`` (default) -- the Gram form (five iterations on m x m matrices with
one rebuild of X, ``mmuon_ns_plan``) for bf16 groups whose padded long side is
at least twice the short side, the three-product chain elsewhere;
``"standard"`` -- the three-product chain ``A = XX^T, P = aI + bA + cA^2,
X = PX`` for every group.  Both equal the reference's iteration in exact
arithmetic.
"""
from __future__ import annotations

import ctypes as C

import torch

from . import _abi
from .plan import (NORM_CHUNK, NS_COEFFS, NS_STEPS, AdamPlanner, MuonPlanner, NormPlanner, adamw_scalars,
                   run_newton_schulz)

_COEFFS = (C.c_float * 3)(*NS_COEFFS)


def _require_gpu(t: torch.Tensor) -> None:
    if not t.is_cuda:
        raise RuntimeError("MonarchMuonOptimizer (MI355X) needs parameters on a ROCm GPU; "
                           f"got a tensor on {t.device}")


class MonarchMuonOptimizer(torch.optim.Optimizer):
    """Muon with batched Newton-Schulz over Monarch blocks + embedded AdamW.

    Group 0 (``update_type="muon"``): 3-D Monarch factors ``(nblocks, rows, cols)``.
    Group 1 (``update_type="adamw"``): every other parameter.
    """

    def __init__(self, muon_params, adamw_params, *, lr: float = 5e-3, momentum: float = 0.95,
                 adamw_betas: tuple = (0.9, 0.95), adamw_weight_decay: float = 0.1,
                 adamw_eps: float = 1e-8, ns_dtype: torch.dtype | None = torch.bfloat16,
                 ns_form: str = "auto"):
        muon_params = list(muon_params)
        adamw_params = list(adamw_params)
        defaults = dict(lr=lr)
        param_groups = [
            {"params": muon_params, "update_type": "muon", "momentum": momentum},
            {"params": adamw_params, "update_type": "adamw", "betas": adamw_betas,
             "weight_decay": adamw_weight_decay, "eps": adamw_eps},
        ]
        super().__init__(param_groups, defaults)
        if ns_dtype not in (torch.bfloat16, torch.float32, None):
            raise ValueError("ns_dtype must be torch.bfloat16, torch.float32 or None")
        self.ns_dtype = ns_dtype
        if ns_form not in ("auto", "standard"):
            raise ValueError('ns_form must be "auto" or "standard"')
        self.ns_form = ns_form
        self._ns_flags = _abi.NS_STANDARD if ns_form == "standard" else 0
        self._muon_planner = MuonPlanner()
        self._adam_planner = AdamPlanner()
        self._norm_planner = NormPlanner()
        self._clip = None    # device clipping coefficient for the next step (clip_grad_norm_)

    # ------------------------------------------------------------------
    @torch.no_grad()
    def step(self, closure=None):
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        try:
            for group in self.param_groups:
                lr = group["lr"]
                if group["update_type"] == "muon":
                    self._muon_step(group, lr)
                else:
                    self._adamw_step(group, lr)
        finally:
            self._clip = None  # a clipping coefficient applies to one step
        return loss

    def _grad_scale(self):
        return self._clip.data_ptr() if self._clip is not None else None

    @torch.no_grad()
    def clip_grad_norm_(self, max_norm: float, norm_type: float = 2.0,
                        error_if_nonfinite: bool = False) -> torch.Tensor:
        """``torch.nn.utils.clip_grad_norm_`` over this optimizer's parameters,
        folded into the next ``step()``.

        The reference clips right before the step
        (``pretrain/src/optim/base.py:121-122``:
        ``torch.nn.utils.clip_grad_norm_(model.parameters(), grad_clip)``, then
        ``opt.step()``).  Here the per-tensor norms, their norm and the
        coefficient ``min(max_norm / (total + 1e-6), 1)`` are computed on the
        device, rounded to the gradients' dtype where torch rounds them, and the
        next ``step()`` reads every gradient as ``dtype(g * coef)`` -- the value
        torch's in-place rescale leaves in ``p.grad``.  The gradients are not
        rewritten, so the rescale pass over them is saved, and nothing
        synchronises with the host.  Returns the total norm (0-dim tensor in the
        gradients' dtype, on the device).  The 2-norm only; every gradient on one
        device, in one dtype.
        """
        if float(norm_type) != 2.0:
            raise NotImplementedError("the fused clip_grad_norm_ computes the 2-norm only")
        grads = [p.grad for group in self.param_groups for p in group["params"] if p.grad is not None]
        if not grads:
            self._clip = None
            return torch.tensor(0.0)
        for g in grads:
            _require_gpu(g)
        grads = [g if g.is_contiguous() else g.contiguous() for g in grads]
        nl = self._norm_planner.plan(grads)
        args = _abi.GradNormArgs(tensors=nl.tensors.data_ptr(), chunks=nl.chunks.data_ptr(),
                                 first_chunk=nl.first_chunk.data_ptr(), nchunks=nl.nchunks, ntensors=nl.ntensors,
                                 chunk_elems=NORM_CHUNK, grad_dtype=_abi.dtype_code(nl.dtype),
                                 max_norm=float(max_norm), partial=nl.partial.data_ptr(), norms=nl.norms.data_ptr(),
                                 total=nl.total.data_ptr(), coef=nl.coef.data_ptr())
        _abi.check(_abi.lib().mmuon_grad_clip_coef(C.byref(args), _abi.stream_handle(grads[0].device)),
                   "mmuon_grad_clip_coef")
        total = nl.total.to(nl.dtype, copy=True).reshape(())  # the value is exact in the gradients' dtype
        if error_if_nonfinite and not bool(torch.isfinite(total)):
            raise RuntimeError(f"The total norm of order {float(norm_type)} for gradients from `parameters` is "
                               "non-finite, so it cannot be clipped. To disable this error and scale the gradients "
                               "by the non-finite norm anyway, set `error_if_nonfinite=False`")
        self._clip = nl.coef
        return total

    def zero_grad(self, set_to_none: bool = True) -> None:
        self._clip = None  # the coefficient belongs to the gradients being dropped
        super().zero_grad(set_to_none=set_to_none)

    def release_workspace(self) -> None:
        """Drop the cached Newton-Schulz workspaces and launch tables."""
        self._muon_planner.release()
        self._adam_planner.release()
        self._norm_planner.release()

    # ------------------------------------------------------------------
    # Muon (membench :134-170, pretrain :133-165)
    # ------------------------------------------------------------------
    def _get_momentum_buffer(self, param: torch.Tensor) -> torch.Tensor:
        state = self.state[param]
        if "momentum_buffer" not in state:
            state["momentum_buffer"] = torch.zeros_like(param, memory_format=torch.contiguous_format)
        return state["momentum_buffer"]

    def _muon_inputs(self, group):
        params = [p for p in group["params"] if p.grad is not None]
        for p in params:
            _require_gpu(p)
        grads = [p.grad if p.grad.is_contiguous() else p.grad.contiguous() for p in params]
        return params, grads

    def _muon_step(self, group: dict, lr: float) -> None:
        params, grads = self._muon_inputs(group)
        if not params:
            return
        bufs = [self._get_momentum_buffer(p) for p in params]
        self._muon_planner.plan(params, grads, bufs, self.ns_dtype)
        momentum = float(group["momentum"])
        lib = _abi.lib()
        gscale = self._grad_scale()

        def pack(gl, stream):
            gl.struct.grad_scale = gscale
            _abi.check(lib.mmuon_momentum_pack(C.byref(gl.struct), momentum, stream), "mmuon_momentum_pack")

        run_newton_schulz(self._muon_planner.units, lib, _COEFFS, lr, self._ns_flags, NS_STEPS,
                          lambda gl: _abi.stream_handle(gl.key[0]), pack)

    # ------------------------------------------------------------------
    # AdamW (membench :176-208; pretrain :171-201 keeps a step per tensor)
    # ------------------------------------------------------------------
    def _adam_states(self, params):
        for p in params:
            state = self.state[p]
            if len(state) == 0:
                state["step"] = 0
                state["exp_avg"] = torch.zeros_like(p, memory_format=torch.contiguous_format)
                state["exp_avg_sq"] = torch.zeros_like(p, memory_format=torch.contiguous_format)
            state["step"] += 1

    def _adamw_step(self, group: dict, lr: float) -> None:
        params = [p for p in group["params"] if p.grad is not None]
        if not params:
            return
        for p in params:
            _require_gpu(p)
        self._adam_states(params)
        grads = [p.grad if p.grad.is_contiguous() else p.grad.contiguous() for p in params]
        ms = [self.state[p]["exp_avg"] for p in params]
        vs = [self.state[p]["exp_avg_sq"] for p in params]
        beta1, beta2 = group["betas"]
        if self.ns_dtype is None:
            steps = [self.state[p]["step"] for p in params]        # pretrain: per tensor
        else:
            steps = [self.state[params[0]]["step"]] * len(params)  # membench :192
        self._launch_adamw(params, grads, ms, vs, steps, lr, beta1, beta2, group["eps"],
                           group["weight_decay"])

    def _launch_adamw(self, params, grads, ms, vs, steps, lr, beta1, beta2, eps, wd, fp8_meta=None, fresh=None):
        """``fresh`` (FP8 states): per tensor, whether its moments are created
        in this step (they start at zero in the parameter dtype)."""
        kinds = [(s, bool(fresh[i]) if fresh is not None else False) for i, s in enumerate(steps)]
        launches = self._adam_planner.plan(params, grads, ms, vs, fp8_meta)
        lib = _abi.lib()
        for al in launches:
            ks = {kinds[i] for i in al.members}
            if len(ks) != 1:
                # tensors whose step counts (or state ages) differ: one launch per kind
                self._adamw_split(al, params, grads, ms, vs, kinds, lr, beta1, beta2, eps, wd, fp8_meta)
                continue
            step, new = ks.pop()
            self._adamw_one(lib, al, step, lr, beta1, beta2, eps, wd, have_state=not new)

    def _adamw_one(self, lib, al, step, lr, beta1, beta2, eps, wd, have_state=True):
        args = _abi.AdamWArgs(tensors=al.tensors.data_ptr(), chunks=al.chunks.data_ptr(), nchunks=al.nchunks,
                              chunk_elems=al.chunk, param_dtype=_abi.dtype_code(al.pd),
                              grad_dtype=_abi.dtype_code(al.gd), state_dtype=_abi.dtype_code(al.sd),
                              grad_scale=self._grad_scale(), **adamw_scalars(lr, beta1, beta2, eps, wd, step))
        stream = _abi.stream_handle(al.tensors.device)
        if al.fp8 is not None:
            _abi.check(lib.mmuon_adamw_fp8(C.byref(args), C.cast(al.fp8.data_ptr(), C.POINTER(_abi.AdamWFp8Tensor)),
                                           int(have_state), _abi.dtype_code(al.vd), float(self.expand_min), stream),
                       "mmuon_adamw_fp8")
        else:
            _abi.check(lib.mmuon_adamw(C.byref(args), stream), "mmuon_adamw")

    def _adamw_split(self, al, params, grads, ms, vs, kinds, lr, beta1, beta2, eps, wd, fp8_meta):
        lib = _abi.lib()
        by_kind: dict = {}
        for i in al.members:
            by_kind.setdefault(kinds[i], []).append(i)
        for (step, new), idx in by_kind.items():
            sub = AdamPlanner().plan([params[i] for i in idx], [grads[i] for i in idx], [ms[i] for i in idx],
                                     [vs[i] for i in idx], [fp8_meta[i] for i in idx] if fp8_meta else None)
            for sl in sub:
                self._adamw_one(lib, sl, step, lr, beta1, beta2, eps, wd, have_state=not new)

    # ------------------------------------------------------------------
    # optional per-launch timing (bench.py): hipEvents on the launch stream
    # ------------------------------------------------------------------


# ---------------------------------------------------------------------------
# FP8 optimizer states (coat_state_muon.py:117-151)
# ---------------------------------------------------------------------------
STATES = {"momentum_buffer": True, "exp_avg": True, "exp_avg_sq": False}   # name -> signed
_FP8 = {"E4M3": torch.float8_e4m3fn, "E5M2": torch.float8_e5m2}          # coat_state_muon.py:17
_META = ("scale", "expand", "sqrt_minmax")


class QuantizationConfig:
    """The optimizer-state fields of COAT's ``QuantizationConfig``
    (``third_party/coat/utils/_fp8_quantization_config.py:20-26``)."""

    def __init__(self, first_order_expansion="true", second_order_expansion="true",
                 first_order_bit="E4M3", second_order_bit="E4M3", qgroup_size=128, expand_min=16, **_):
        self.first_order_expansion = first_order_expansion
        self.second_order_expansion = second_order_expansion
        self.first_order_bit = first_order_bit
        self.second_order_bit = second_order_bit
        self.qgroup_size = qgroup_size
        self.expand_min = expand_min


class CoatStateMonarchMuon(MonarchMuonOptimizer):
    """Every optimizer state stored as FP8 (``first_order_bit`` for the momentum
    and ``exp_avg``, ``second_order_bit`` for ``exp_avg_sq``: E4M3 or E5M2) in
    groups of 128 of the flattened tensor with dynamic range expansion
    (``expand_min``); each step dequantizes, updates and requantizes inside the
    fused kernels.  A Monarch factor whose blocks hold a multiple of 128
    elements is updated in place (no fp32 copy of the momentum); one whose
    groups straddle its blocks takes the reference's own sequence over the
    whole parameter: dequantize to a (cached) fp32 buffer, the plain step,
    quantize back."""

    def __init__(self, *args, qargs, **kwargs):
        if qargs.qgroup_size != 128:
            raise AssertionError("COAT's optimizer kernels use groups of 128")
        if qargs.first_order_expansion not in ("expand", "true") or qargs.second_order_expansion not in ("expand", "true"):
            raise AssertionError("only the dynamic-range-expansion codec is supported")
        for bit in (qargs.first_order_bit, qargs.second_order_bit):
            if bit not in _FP8:
                raise KeyError(f"FP8 state format {bit!r} (E4M3 or E5M2)")
        emin = float(qargs.expand_min)
        if not (emin > 0 and emin < float("inf")):
            raise ValueError(f"expand_min must be positive (got {qargs.expand_min})")
        self.dtypes = {name: _FP8[qargs.first_order_bit] for name in ("momentum_buffer", "exp_avg")}
        self.dtypes["exp_avg_sq"] = _FP8[qargs.second_order_bit]
        self.expand_min = qargs.expand_min
        self._ragged = {}   # parameter -> cached momentum buffer of the straddling-group path
        super().__init__(*args, **kwargs)

    def _ensure_fp8(self, state, name, like):
        """FP8 payload + metadata for ``state[name]`` in this optimizer's format;
        a missing state starts as exact zeros (codes 0 decode to 0 whatever the
        metadata)."""
        fmt = self.dtypes[name]
        groups = (like.numel() + 127) // 128
        cur = state.get(name)
        if cur is None:
            state[name] = torch.zeros(like.shape, dtype=fmt, device=like.device)
            for key in _META:
                state[f"{key}_{name}"] = torch.ones(groups, dtype=torch.float32, device=like.device)
        for key in _META:
            t = state[f"{key}_{name}"]
            if t.dtype != torch.float32:
                state[f"{key}_{name}"] = t.to(torch.float32)
        cur = state[name]
        if cur.dtype != fmt:
            # a floating state (e.g. restored without its FP8 dtype), or codes of
            # the other FP8 format: quantize its value in this format
            if cur.dtype in _abi.FP8_DTYPES:
                value = torch.empty(like.shape, dtype=torch.float32, device=like.device)
                _abi.fp8_dequantize(cur.contiguous(), *self._meta(state, name), value, signed=STATES[name],
                                    fmt=cur.dtype)
            else:
                value = cur.detach().to(torch.float32).contiguous()
            codes = torch.empty(like.shape, dtype=fmt, device=like.device)
            meta = [torch.empty(groups, dtype=torch.float32, device=like.device) for _ in range(3)]
            _abi.fp8_quantize(value, codes, *meta, signed=STATES[name], fmt=fmt, expand_min=self.expand_min)
            state[name] = codes
            for key, t in zip(_META, meta):
                state[f"{key}_{name}"] = t
        return state[name]

    def _meta(self, state, name):
        return tuple(state[f"{key}_{name}"] for key in _META)

    def _ragged_buffer(self, p, dtype, codes, meta, have_state):
        """The momentum of a parameter whose 128-groups straddle its blocks, as
        the wrapped step sees it (coat_state_muon.py:128-132): the dequantized
        fp32 tensor, or zeros in the parameter dtype when the step creates it.
        The buffer is kept between steps (same shape and dtype)."""
        buf = self._ragged.get(p)
        if buf is None or buf.dtype != dtype or buf.shape != p.shape:
            buf = self._ragged[p] = torch.empty(p.shape, dtype=dtype, device=p.device)
        if have_state:
            _abi.fp8_dequantize(codes, *meta, buf, signed=True, fmt=codes.dtype)
        else:
            buf.zero_()
        return buf

    def release_workspace(self) -> None:
        super().release_workspace()
        self._ragged = {}

    def _muon_step(self, group: dict, lr: float) -> None:
        params, grads = self._muon_inputs(group)
        if not params:
            return
        # the wrapped step sees a dequantized (fp32) momentum, or one it creates
        # with zeros_like(param) in the parameter dtype on a parameter's first
        # step: that dtype keys the grouping and, with ns_dtype=None, is the
        # Newton-Schulz dtype
        name = "momentum_buffer"
        have = ["momentum_buffer" in self.state[p] for p in params]
        key_dtypes = [torch.float32 if h else p.dtype for p, h in zip(params, have)]
        bufs, metas, ragged = [], [], []
        for p, h, kd in zip(params, have, key_dtypes):
            if p.dim() != 3:
                raise ValueError(f"Muon parameters must be 3-D (nblocks, rows, cols); got shape {tuple(p.shape)}")
            st = self.state[p]
            codes = self._ensure_fp8(st, name, p)
            if (p.shape[1] * p.shape[2]) % 128 == 0:
                bufs.append(codes)
                metas.append(self._meta(st, name))
            else:
                buf = self._ragged_buffer(p, kd, codes, self._meta(st, name), h)
                bufs.append(buf)
                metas.append(None)
                ragged.append((p, buf))
        self._muon_planner.plan(params, grads, bufs, self.ns_dtype, fp8_meta=metas, key_dtypes=key_dtypes)
        momentum = float(group["momentum"])
        lib = _abi.lib()
        gscale = self._grad_scale()
        emin = float(self.expand_min)

        def pack(gl, stream):
            gl.struct.grad_scale = gscale
            if gl.struct.buf_dtype in (_abi.F8E4M3, _abi.F8E5M2):
                _abi.check(lib.mmuon_fp8_momentum_pack(C.byref(gl.struct), momentum, 1, emin, stream),
                           "mmuon_fp8_momentum_pack")
            else:
                _abi.check(lib.mmuon_momentum_pack(C.byref(gl.struct), momentum, stream), "mmuon_momentum_pack")

        run_newton_schulz(self._muon_planner.units, lib, _COEFFS, lr, self._ns_flags, NS_STEPS,
                          lambda gl: _abi.stream_handle(gl.key[0]), pack)
        for p, buf in ragged:   # quantize_ (coat_state_muon.py:134-138) over the whole parameter
            st = self.state[p]
            value = buf if buf.dtype == torch.float32 else buf.to(torch.float32)
            _abi.fp8_quantize(value, st[name], *self._meta(st, name), signed=True, fmt=st[name].dtype,
                              expand_min=self.expand_min)

    def _adamw_step(self, group: dict, lr: float) -> None:
        params = [p for p in group["params"] if p.grad is not None]
        if not params:
            return
        fresh = []
        for p in params:
            _require_gpu(p)
            state = self.state[p]
            # moments created in this step start at zero in the parameter dtype
            # (zeros_like(param) in the wrapped step) and are rounded to it
            fresh.append("exp_avg" not in state)
            if "step" not in state:
                state["step"] = 0
            state["step"] += 1
            self._ensure_fp8(state, "exp_avg", p)
            self._ensure_fp8(state, "exp_avg_sq", p)
        grads = [p.grad if p.grad.is_contiguous() else p.grad.contiguous() for p in params]
        ms = [self.state[p]["exp_avg"] for p in params]
        vs = [self.state[p]["exp_avg_sq"] for p in params]
        meta = [self._meta(self.state[p], "exp_avg") + self._meta(self.state[p], "exp_avg_sq") for p in params]
        beta1, beta2 = group["betas"]
        if self.ns_dtype is None:
            steps = [self.state[p]["step"] for p in params]
        else:
            steps = [self.state[params[0]]["step"]] * len(params)
        self._launch_adamw(params, grads, ms, vs, steps, lr, beta1, beta2, group["eps"],
                           group["weight_decay"], fp8_meta=meta, fresh=fresh)

    def load_state_dict(self, state_dict):
        # torch.optim casts floating state to the parameter dtype; put the FP8
        # payloads (exact in any wider float) and fp32 metadata back.
        saved = {key: {name: value.dtype for name, value in entry.items() if name in STATES}
                 for key, entry in state_dict["state"].items()}
        super().load_state_dict(state_dict)
        params = [p for group in self.param_groups for p in group["params"]]
        for key, dtypes in saved.items():
            p = params[key]
            state = self.state[p]
            entry = state_dict["state"][key]
            for name, dtype in dtypes.items():
                state[name] = state[name].to(dtype)
                for meta in _META:
                    mk = f"{meta}_{name}"
                    if mk in entry:
                        # the saved fp32 metadata itself (torch's cast to a bf16
                        # parameter dtype would round it)
                        state[mk] = entry[mk].detach().to(device=p.device, dtype=torch.float32).clone()
