"""torch-CPU restatement of ``MonarchMuonOptimizer.step()`` -- test infrastructure.

Reference copies restated here (all paths relative to the reference repo):

* ``membench/src/models/monarch/monarch_muon.py`` -- momentum in the buffer
  dtype, cast of each same-shape stack to bf16 (``:162-163``), Newton-Schulz
  in bf16, cast back and ``_foreach_add_`` apply (``:140-170``), foreach AdamW
  (``:176-208``).  This is the variant behind the published step time.
* ``pretrain/src/models/monarch/monarch_muon.py`` -- identical grouping, but no
  bf16 cast: Newton-Schulz runs in the buffer dtype (``:139-165``); per-tensor
  AdamW (``:171-201``).

The op sequence below follows the reference line by line on purpose: the
oracle must round where the reference rounds (every torch op rounds to its
tensor dtype).  Pinning: ``tests/test_oracle.py`` checks the Newton-Schulz
restatement against the SVD known answer and the orthogonal-invariance
identities, the momentum/apply arithmetic against fp64 brute force, the AdamW
against ``torch.optim.AdamW`` and the grouping against the closed-form block
inventory; ``tests/golden`` holds vectors written by the reference itself.
"""
from __future__ import annotations

import math
from collections import OrderedDict

import torch

NS_COEFFS = (3.4445, -4.7750, 2.0315)   # monarch_muon.py:47
NS_STEPS = 5                            # monarch_muon.py:45
NS_EPS = 1e-7                           # monarch_muon.py:39


def newton_schulz_batched(B: torch.Tensor) -> torch.Tensor:
    """Restates ``_newton_schulz_batched`` (membench and pretrain ``:36-50``).

    Frobenius-normalise each block, transpose tall blocks, five quintic steps
    written exactly as the reference writes them (four products per step, with
    Python's left-to-right ``*``/``@`` association), transpose back.
    """
    norms = B.norm(p="fro", dim=(-2, -1), keepdim=True)
    B = B / (norms + NS_EPS)
    transposed = B.shape[-2] > B.shape[-1]
    if transposed:
        B = B.transpose(-2, -1)
    # On a GPU (tests run this restatement there to get torch's GPU rounding of
    # Python scalars) every right operand is made contiguous: same values, and
    # batched bf16 products with a transposed right operand are avoided.
    lay = (lambda t: t.contiguous()) if B.is_cuda else (lambda t: t)
    B = lay(B)
    a, b, c = NS_COEFFS
    for _ in range(NS_STEPS):
        BBt = B @ lay(B.transpose(-2, -1))
        # reference: 3.4445 * B - 4.7750 * BBt @ B + 2.0315 * (BBt @ BBt) @ B
        B = a * B - (-b) * BBt @ B + c * (BBt @ BBt) @ B
    if transposed:
        B = B.transpose(-2, -1)
    return B


def group_blocks(params, bufs):
    """Restates the bucketing of ``_muon_step`` (membench ``:153-157``).

    Key ``(device, dtype, rows, cols)`` of the momentum buffer, dict insertion
    order = first appearance in parameter order.  Returns an OrderedDict
    key -> list of (param_index, param, buf).
    """
    grouped: "OrderedDict[tuple, list]" = OrderedDict()
    for i, (p, buf) in enumerate(zip(params, bufs)):
        key = (buf.device, buf.dtype, buf.shape[1], buf.shape[2])
        grouped.setdefault(key, []).append((i, p, buf))
    return grouped


class ReferenceMonarchMuon(torch.optim.Optimizer):
    """CPU restatement of ``MonarchMuonOptimizer`` (membench ``:57-208``).

    ``variant="membench"`` casts each stack to bf16 before Newton-Schulz (the
    bf16 oracle); ``variant="pretrain"`` keeps the buffer dtype (the fp32
    oracle).  Constructor, param groups and state keys equal the reference's
    (``:79-108``).
    """

    def __init__(self, muon_params, adamw_params, *, lr=5e-3, momentum=0.95,
                 adamw_betas=(0.9, 0.95), adamw_weight_decay=0.1, adamw_eps=1e-8,
                 variant="membench"):
        if variant not in ("membench", "pretrain"):
            raise ValueError(variant)
        self.variant = variant
        defaults = dict(lr=lr)
        groups = [
            {"params": list(muon_params), "update_type": "muon", "momentum": momentum},
            {"params": list(adamw_params), "update_type": "adamw", "betas": adamw_betas,
             "weight_decay": adamw_weight_decay, "eps": adamw_eps},
        ]
        super().__init__(groups, defaults)

    @torch.no_grad()
    def step(self, closure=None):
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        for group in self.param_groups:
            lr = group["lr"]
            if group["update_type"] == "muon":
                self._muon_step(group, lr)
            else:
                self._adamw_step(group, lr)
        return loss

    def _get_momentum_buffer(self, param):
        state = self.state[param]
        if "momentum_buffer" not in state:
            state["momentum_buffer"] = torch.zeros_like(param)
        return state["momentum_buffer"]

    def _muon_step(self, group, lr):
        momentum = group["momentum"]
        params = [p for p in group["params"] if p.grad is not None]
        if not params:
            return
        bufs = [self._get_momentum_buffer(p) for p in params]
        grads = [p.grad for p in params]
        if self.variant == "membench":
            torch._foreach_mul_(bufs, momentum)         # membench :150
            torch._foreach_add_(bufs, grads)            # membench :151
        else:
            for buf, grad in zip(bufs, grads):          # pretrain :147-148
                buf.mul_(momentum).add_(grad)
        for (_, _, a, b), items in group_blocks(params, bufs).items():
            merged = torch.cat([buf for _, _, buf in items], dim=0)
            if self.variant == "membench" and merged.dtype != torch.bfloat16:
                merged = merged.to(torch.bfloat16)       # membench :162-163
            ortho = newton_schulz_batched(merged)
            if ortho.dtype != items[0][2].dtype:
                ortho = ortho.to(items[0][2].dtype)      # membench :165-166
            scale = (a / b) ** 0.5
            if self.variant == "membench":
                updates = list(ortho.split([buf.shape[0] for _, _, buf in items], dim=0))
                torch._foreach_add_([p.data for _, p, _ in items], updates, alpha=-lr * scale)
            else:
                offset = 0                               # pretrain :160-165
                for _, p, buf in items:
                    n = buf.shape[0]
                    p.data.add_(ortho[offset:offset + n], alpha=-lr * scale)
                    offset += n

    def _adamw_step(self, group, lr):
        beta1, beta2 = group["betas"]
        weight_decay = group["weight_decay"]
        eps = group["eps"]
        params = [p for p in group["params"] if p.grad is not None]
        if not params:
            return
        if self.variant == "pretrain":                   # pretrain :176-201
            for p in params:
                state = self.state[p]
                if len(state) == 0:
                    state["step"] = 0
                    state["exp_avg"] = torch.zeros_like(p)
                    state["exp_avg_sq"] = torch.zeros_like(p)
                state["step"] += 1
                step = state["step"]
                ea, eas, g = state["exp_avg"], state["exp_avg_sq"], p.grad
                if weight_decay > 0:
                    p.data.mul_(1.0 - lr * weight_decay)
                ea.mul_(beta1).add_(g, alpha=1.0 - beta1)
                eas.mul_(beta2).addcmul_(g, g, value=1.0 - beta2)
                bc1 = 1.0 - beta1 ** step
                bc2 = 1.0 - beta2 ** step
                denom = (eas.sqrt() / math.sqrt(bc2)).add_(eps)
                p.data.addcdiv_(ea, denom, value=-(lr / bc1))
            return
        for p in params:                                 # membench :184-190
            state = self.state[p]
            if len(state) == 0:
                state["step"] = 0
                state["exp_avg"] = torch.zeros_like(p)
                state["exp_avg_sq"] = torch.zeros_like(p)
            state["step"] += 1
        step = self.state[params[0]]["step"]
        grads = [p.grad for p in params]
        exp_avgs = [self.state[p]["exp_avg"] for p in params]
        exp_avg_sqs = [self.state[p]["exp_avg_sq"] for p in params]
        if weight_decay > 0:
            torch._foreach_mul_([p.data for p in params], 1.0 - lr * weight_decay)
        torch._foreach_mul_(exp_avgs, beta1)
        torch._foreach_add_(exp_avgs, grads, alpha=1.0 - beta1)
        torch._foreach_mul_(exp_avg_sqs, beta2)
        torch._foreach_addcmul_(exp_avg_sqs, grads, grads, value=1.0 - beta2)
        bc1 = 1.0 - beta1 ** step
        bc2 = 1.0 - beta2 ** step
        denom = torch._foreach_sqrt(exp_avg_sqs)
        torch._foreach_div_(denom, math.sqrt(bc2))
        torch._foreach_add_(denom, eps)
        torch._foreach_addcdiv_([p.data for p in params], exp_avgs, denom, value=-lr / bc1)


def newton_schulz_ortho(stack: torch.Tensor, ns_dtype=torch.bfloat16) -> torch.Tensor:
    """Newton-Schulz of a ``(N, rows, cols)`` stack as the step performs it:
    cast to ``ns_dtype`` (membench ``:162-163``; ``None`` keeps the dtype as
    the pretrain copy does), then ``newton_schulz_batched``."""
    x = stack if ns_dtype is None or stack.dtype == ns_dtype else stack.to(ns_dtype)
    return newton_schulz_batched(x)


# ---------------------------------------------------------------------------
# FP8 optimizer states (pretrain/src/models/monarch/coat_state_muon.py:117-139)
# ---------------------------------------------------------------------------
FP8_STATES = {"momentum_buffer": True, "exp_avg": True, "exp_avg_sq": False}   # name -> signed
FP8_FORMATS = {torch.float8_e4m3fn: "E4M3", torch.float8_e5m2: "E5M2"}          # coat_state_muon.py:17


def dequantize_state(state: dict, name: str, signed: bool) -> torch.Tensor:
    """Restates ``dequantize`` (``coat_state_muon.py:94-100``): the FP8 payload
    ``state[name]`` (e4m3fn or e5m2, decoded as its dtype) and its per-128
    metadata -> an fp32 tensor of the same shape on the same device."""
    data = state[name]
    meta = [state[f"{key}_{name}"].detach().cpu().to(torch.float32).numpy() for key in ("scale", "expand",
                                                                                        "sqrt_minmax")]
    from . import codec
    out = codec.dequantize(data.detach().cpu().view(torch.uint8).numpy().reshape(-1), *meta, signed,
                           FP8_FORMATS[data.dtype])
    return torch.from_numpy(out).reshape(data.shape).to(data.device)


def quantize_state(state: dict, name: str, value: torch.Tensor, signed: bool,
                   dtype: torch.dtype = torch.float8_e4m3fn, expand_min: float = 16) -> None:
    """Restates ``quantize_`` (``coat_state_muon.py:103-114``): store ``value``
    (any float dtype; the kernel loads it as fp32) as ``dtype`` codes (its
    ``finfo.max`` is the codec's fp8_max) plus fp32
    ``scale_/expand_/sqrt_minmax_<name>``."""
    from . import codec
    codes, scale, expand, smm = codec.quantize(value.detach().to(torch.float32).cpu().numpy().reshape(-1), signed,
                                               FP8_FORMATS[dtype], expand_min)
    dev = value.device
    state[name] = torch.from_numpy(codes).view(dtype).reshape(value.shape).to(dev)
    for key, t in zip(("scale", "expand", "sqrt_minmax"), (scale, expand, smm)):
        state[f"{key}_{name}"] = torch.from_numpy(t).to(dev)


class ReferenceCoatStateMonarchMuon(ReferenceMonarchMuon):
    """CPU restatement of ``CoatStateMonarchMuon.step`` (``coat_state_muon.py:126-139``).

    Every state present before the step is dequantized to fp32, the unchanged
    step runs (``variant`` selects the copy it wraps: ``pretrain`` is the
    reference's own class; ``membench`` wraps the bf16-Newton-Schulz copy the
    same way), and every state of a parameter that had a gradient is quantized
    back.  A state created during the step is created by the wrapped copy with
    ``zeros_like(param)`` -- in the PARAMETER dtype -- so on a parameter's first
    step the momentum, the Newton-Schulz input (pretrain copy) and the AdamW
    moments are computed in that dtype and quantized from it; on later steps
    the dequantized states are fp32."""

    keep_values = False   # tests: keep each state's value before it is quantized
    # per state, the FP8 dtype it is stored in, and the codec's expand_min
    # (coat_state_muon.py:121-123: first_order_bit for the momentum and exp_avg,
    # second_order_bit for exp_avg_sq; COAT's defaults)
    dtypes = {"momentum_buffer": torch.float8_e4m3fn, "exp_avg": torch.float8_e4m3fn,
              "exp_avg_sq": torch.float8_e4m3fn}
    expand_min = 16

    @torch.no_grad()
    def step(self, closure=None):
        active = [p for group in self.param_groups for p in group["params"] if p.grad is not None]
        for p in active:
            state = self.state[p]
            for name, signed in FP8_STATES.items():
                if name in state:
                    state[name] = dequantize_state(state, name, signed)
        loss = super().step(closure)
        self.values = {}
        for p in active:
            state = self.state[p]
            for name, signed in FP8_STATES.items():
                if name in state:
                    value = state.pop(name)
                    if self.keep_values:
                        self.values.setdefault(p, {})[name] = value
                    quantize_state(state, name, value, signed, self.dtypes[name], self.expand_min)
        return loss
