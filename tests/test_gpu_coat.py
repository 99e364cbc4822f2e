"""GPU parity of the FP8-state optimizer ``CoatStateMonarchMuon`` against the
oracle's restatement of the reference wrapper
(``pretrain/src/models/monarch/coat_state_muon.py:117-139``: dequantize every
state to fp32, run the unchanged step, quantize every state back; a state the
step creates starts as ``zeros_like(param)`` in the parameter dtype).

Each step is compared from identical inputs: before every step after the
first, the oracle takes the GPU's parameters and FP8 states.  The oracle's
torch ops run on the GPU (torch's GPU kernels keep Python scalars in fp32 when
they scale a bf16 tensor, its CPU kernels round some of them to bf16 first);
its codec is the numpy restatement.

Bars, per step:
- weights within 1e-2 relative Frobenius per block when they are bf16, within
  1e-5 when they are fp32 with fp32 Newton-Schulz (the north star's bars);
- state codes against ``codec.quantize`` of the oracle's value before
  quantization: at most 1 e4m3 code apart, on fewer than 0.5% of the elements
  (the GPU's powers are 2^(y log2 x) with the hardware exp2/log2, about 1e-6
  relative, so values next to an e4m3 rounding boundary may land on the
  neighbouring code); expansion exactly equal on at least 99.9% of the groups
  (``floor`` of a log ratio: a group on a step may take the other one); the
  group maximum the metadata encode, sqrt_minmax (448 scale)^(1/expand),
  within 1e-5 relative (scale and sqrt_minmax separately also follow the
  group's smallest non-zero |value|, where the momentum update mu*old + g can
  cancel and turn the 1e-6 difference of the two decoders into a large
  relative one; neither the codes nor the decoded values depend on it); and on
  every element, our codes decode with our metadata to the value within the
  e4m3 round-trip bound plus 4e-6 of the group maximum (the same
  cancellation, seen on the element itself).
"""
import numpy as np
import pytest
import torch

from monarch_muon_amd import CoatStateMonarchMuon, QuantizationConfig
from oracle import codec
from oracle.step import FP8_STATES, ReferenceCoatStateMonarchMuon, ReferenceMonarchMuon, dequantize_state
from test_gpu_parity import BF16_TOL, DEV, F32_TOL, _workload_params, blocks_rel

pytestmark = pytest.mark.gpu


def _params(draws, dtype):
    muon, adamw = [], []
    for _, is_muon, W, G, _ in draws:
        p = W.to(dtype).to(DEV).requires_grad_(True)
        p.grad = G.to(dtype).to(DEV)
        (muon if is_muon else adamw).append(p)
    return muon, adamw


def _sync(gparams, gopt, cparams, copt):
    """The oracle starts this step from the GPU's parameters and states."""
    with torch.no_grad():
        for p, q in zip(gparams, cparams):
            q.copy_(p)
            copt.state[q] = {k: (v.clone() if torch.is_tensor(v) else v) for k, v in gopt.state[p].items()}


FMT = {torch.float8_e4m3fn: ("E4M3", 448.0, 2.0 ** -4, 2.0 ** -10),
       torch.float8_e5m2: ("E5M2", 57344.0, 2.0 ** -3, 2.0 ** -17)}   # name, max, relative and subnormal rounding


def _compare_codes(st, name, value, signed, blocks=None, stats=None, expand_min=16):
    """GPU state ``st[name]`` (codes + metadata, in the state's FP8 format)
    against ``codec.quantize(value)``.  ``blocks``: indices of the
    leading-dimension slices to compare (each a whole number of 128-groups), or
    None for all."""
    fmt, fmax, rel_q, abs_q = FMT[st[name].dtype]
    codes = st[name].view(torch.uint8)
    meta = [st[f"{k}_{name}"] for k in ("scale", "expand", "sqrt_minmax")]
    value = value.detach().float()
    if blocks is not None:
        per = value[0].numel()
        gpb = per // 128
        codes = torch.cat([codes[b].reshape(-1) for b in blocks])
        meta = [torch.cat([m[b * gpb:(b + 1) * gpb] for b in blocks]) for m in meta]
        value = torch.cat([value[b].reshape(-1) for b in blocks])
    x = value.cpu().numpy().reshape(-1)
    ref = codec.quantize(x, signed, fmt, expand_min)
    ours = codes.cpu().numpy().reshape(-1)
    sc, ex, smm = (m.cpu().numpy() for m in meta)
    diff = np.abs(ours.astype(np.int32) - ref[0].astype(np.int32))
    ok = ex == ref[2]                              # groups whose expansion agrees
    okel = np.repeat(ok, 128)[:x.size]
    # the decoder sees the metadata only through absmax = smm (fmax scale)^(1/expand)
    # (decode(c) = (c scale)^(1/expand) smm = (c/fmax)^(1/expand) absmax)
    e64 = ex.astype(np.float64)
    amax_ours = smm.astype(np.float64) * (fmax * sc.astype(np.float64)) ** (1.0 / e64)
    amax_ref = ref[3].astype(np.float64) * (fmax * ref[1].astype(np.float64)) ** (1.0 / ref[2].astype(np.float64))
    out = dict(max_code_diff=int(diff[okel].max(initial=0)),
               code_mismatch=float(np.mean(diff[okel] != 0)) if okel.any() else 0.0,
               expand_mismatch=float(np.mean(~ok)) if ok.size else 0.0,
               absmax_rel=float(np.max(np.abs(amax_ours / amax_ref - 1), initial=0)),
               smm_rel_median=float(np.median(np.abs(smm / ref[3] - 1))) if ok.size else 0.0)
    if stats is not None:
        stats.append((name, out))
    assert out["max_code_diff"] <= 1, (name, out)
    assert out["code_mismatch"] < 5e-3, (name, out)
    assert out["expand_mismatch"] <= 1e-3, (name, out)
    assert out["absmax_rel"] <= 1e-5, (name, out)
    # every element: our codes decode (with our metadata) to the value within
    # the format's round-trip bound (q = fmax (|x|/absmax)^expand is kept to
    # 2^-4 relative (e4m3; e5m2 2^-3), 2^-10 (2^-17) absolute when subnormal;
    # the decoder raises to 1/expand)
    dec = codec.dequantize(ours, sc, ex, smm, signed, fmt).astype(np.float64)
    xd = x.astype(np.float64)
    grp = np.arange(x.size) // 128
    amax = np.zeros(ok.size)
    np.maximum.at(amax, grp, np.abs(xd))
    e = ex[grp].astype(np.float64)
    q = fmax * (np.abs(xd) / np.maximum(amax[grp], 1e-300)) ** e
    eq = np.maximum(rel_q, abs_q / np.maximum(q, 1e-300))
    bound = np.maximum(1 - np.clip(1 - eq, 0, None) ** (1.0 / e), (1 + eq) ** (1.0 / e) - 1) + 1e-5
    nz = xd != 0
    # plus an absolute 4e-6 of the group maximum: the two implementations'
    # momenta mu*old + g differ by about 1e-6 of the inputs (the decoders of old
    # differ by that much), which is a large relative difference where the
    # update cancels to a value far below the group maximum
    viol = np.abs(dec - xd) > bound * np.abs(xd) + 4e-6 * amax[grp]
    viol &= nz
    if viol.any():
        idx = np.nonzero(viol)[0][:8]
        rows = [(int(i), float(xd[i]), float(dec[i]), float(q[i]), float(bound[i]), float(e[i]), int(ours[i]),
                 int(ref[0][i]), float(amax[grp[i]])) for i in idx]
        raise AssertionError(f"{name}: {int(viol.sum())} elements decode outside the round-trip bound "
                             f"(index, value, decoded, q, bound, expand, our code, oracle code, group max): {rows}")
    assert np.all(dec[~nz] == 0), (name, out)
    return out


def _weights_bar(dtype, ns_dtype):
    return F32_TOL if dtype == torch.float32 and ns_dtype is None else BF16_TOL


@pytest.mark.parametrize("name,layers,rows", [("toy", None, 256), ("257m-nb2", 1, 512)])
def test_pretrain_fp8_states_three_steps_against_oracle(name, layers, rows):
    """The reference's own FP8-state class: the pretrain copy (Newton-Schulz in
    the momentum dtype: the parameter dtype on the first step, fp32 after)."""
    w, draws = _workload_params(name, layers, rows)
    dtype = w.param_dtype
    gm, ga = _params(draws, dtype)
    cm, ca = _params(draws, dtype)
    gopt = CoatStateMonarchMuon(gm, ga, lr=0.02, momentum=0.95, qargs=QuantizationConfig(), ns_dtype=None)
    copt = ReferenceCoatStateMonarchMuon(cm, ca, lr=0.02, momentum=0.95, variant="pretrain")
    copt.keep_values = True
    tol = _weights_bar(dtype, None)
    for step in range(3):
        if step:
            _sync(gm + ga, gopt, cm + ca, copt)
        copt.step()
        gopt.step()
        torch.cuda.synchronize()
        worst, stats = 0.0, []
        for p, q in zip(gm + ga, cm + ca):
            e = blocks_rel(p, q).max().item()
            worst = max(worst, e)
            assert e <= tol, (step, e)
            for sname, signed in FP8_STATES.items():
                if sname in copt.values.get(q, {}):
                    assert gopt.state[p][sname].dtype == torch.float8_e4m3fn
                    _compare_codes(gopt.state[p], sname, copt.values[q][sname], signed, stats=stats)
        # on the first step the states were created in the parameter dtype
        if step == 0:
            assert all(v.dtype == dtype for d in copt.values.values() for v in d.values())
        else:
            assert all(v.dtype == torch.float32 for d in copt.values.values() for v in d.values())
        mc = max(s["code_mismatch"] for _, s in stats)
        print(f"{name} step {step + 1}: worst weight error {worst:.3e} (bar {tol}), worst code-mismatch "
              f"fraction {mc:.2e}, states compared {len(stats)}")


def test_pretrain_fp8_first_step_newton_schulz_in_param_dtype():
    """bf16 parameters: the reference's first FP8-state step runs Newton-Schulz
    on the bf16 momentum it just created; with fp32 Newton-Schulz the update
    would differ from the oracle's by far more than the bf16-vs-bf16 gap."""
    w, draws = _workload_params("257m-nb2", 1, 64)
    gm, ga = _params(draws, torch.bfloat16)
    gopt = CoatStateMonarchMuon(gm, ga, lr=0.02, momentum=0.95, qargs=QuantizationConfig(), ns_dtype=None)
    gopt.step()
    keys = [gl.key for gl in gopt._muon_planner.groups]
    assert all(k[1] == torch.bfloat16 for k in keys), keys
    assert all(gl.struct.ns_dtype == 1 for gl in gopt._muon_planner.groups)   # MMUON_BF16
    gopt.step()
    assert all(gl.key[1] == torch.float32 and gl.struct.ns_dtype == 0 for gl in gopt._muon_planner.groups)


def test_membench_fp8_states_6p89b_layer_against_oracle():
    """BASELINE's FP8-state configuration on one 6.89B layer (1024 / 2752
    geometry): e4m3 momentum prefilled from N(0, 1e-3), bf16 Newton-Schulz
    (the membench copy wrapped like the reference wraps the pretrain copy).
    The oracle is the wrapper's composition (decode the GPU's states, run the
    unchanged step); codes are compared on one whole block of every Muon
    parameter (the numpy encoder would take minutes on all 80M elements)."""
    w, draws = _workload_params("6.89b-nb4-fp8", layers=1, adamw_rows=64)
    gm, ga = _params(draws, torch.bfloat16)
    cm, ca = _params(draws, torch.bfloat16)
    gopt = CoatStateMonarchMuon(gm, ga, lr=0.02, momentum=0.95, qargs=QuantizationConfig(), ns_dtype=torch.bfloat16)
    bufs = [B for _, is_muon, _, _, B in draws if is_muon]
    for p, b in zip(gm, bufs):
        q, sc, ex, smm = codec.quantize(b.numpy(), True)
        st = gopt.state[p]
        st["momentum_buffer"] = torch.from_numpy(q).view(torch.float8_e4m3fn).reshape(p.shape).to(DEV)
        for key, t in zip(("scale", "expand", "sqrt_minmax"), (sc, ex, smm)):
            st[f"{key}_momentum_buffer"] = torch.from_numpy(t).to(DEV)
    for step in range(2):
        copt = ReferenceMonarchMuon(cm, ca, lr=0.02, momentum=0.95, variant="membench")
        with torch.no_grad():
            for p, q in zip(gm + ga, cm + ca):
                q.copy_(p)
                st = gopt.state[p]
                for sname, signed in FP8_STATES.items():
                    if sname in st:
                        copt.state[q][sname] = dequantize_state(st, sname, signed)
                if "step" in st:
                    copt.state[q]["step"] = st["step"]
        copt.step()
        gopt.step()
        torch.cuda.synchronize()
        stats, worst = [], 0.0
        for i, (p, q) in enumerate(zip(gm, cm)):
            e = blocks_rel(p, q).max().item()
            worst = max(worst, e)
            assert e <= BF16_TOL, (step, i, e)
            _compare_codes(gopt.state[p], "momentum_buffer", copt.state[q]["momentum_buffer"], True,
                           blocks=[i % p.shape[0]], stats=stats)
        for p, q in zip(ga, ca):
            assert blocks_rel(p, q).max() <= BF16_TOL
            for sname, signed in (("exp_avg", True), ("exp_avg_sq", False)):
                assert copt.state[q][sname].dtype == (torch.bfloat16 if step == 0 else torch.float32)
                _compare_codes(gopt.state[p], sname, copt.state[q][sname], signed, stats=stats)
        mc = max(s["code_mismatch"] for _, s in stats)
        print(f"6.89b-nb4-fp8 layer step {step + 1}: worst weight error {worst:.3e}, worst code-mismatch {mc:.2e}")


@pytest.mark.parametrize("first,second,emin", [("E5M2", "E5M2", 16), ("E4M3", "E5M2", 8), ("E5M2", "E4M3", 32)])
def test_fp8_state_formats_and_expand_min_against_oracle(first, second, emin):
    """The formats and expand_min COAT's config exposes
    (``_fp8_quantization_config.py:23-26``): first_order_bit for the momentum and
    exp_avg, second_order_bit for exp_avg_sq (``coat_state_muon.py:121-123``),
    on the toy configuration (pretrain copy, fp32) for three steps."""
    w, draws = _workload_params("toy", None, 256)
    gm, ga = _params(draws, torch.float32)
    cm, ca = _params(draws, torch.float32)
    qa = QuantizationConfig(first_order_bit=first, second_order_bit=second, expand_min=emin)
    gopt = CoatStateMonarchMuon(gm, ga, lr=0.02, momentum=0.95, qargs=qa, ns_dtype=None)
    copt = ReferenceCoatStateMonarchMuon(cm, ca, lr=0.02, momentum=0.95, variant="pretrain")
    f8 = {"E4M3": torch.float8_e4m3fn, "E5M2": torch.float8_e5m2}
    copt.dtypes = {"momentum_buffer": f8[first], "exp_avg": f8[first], "exp_avg_sq": f8[second]}
    copt.expand_min = emin
    copt.keep_values = True
    for step in range(3):
        if step:
            _sync(gm + ga, gopt, cm + ca, copt)
        copt.step()
        gopt.step()
        torch.cuda.synchronize()
        stats = []
        for p, q in zip(gm + ga, cm + ca):
            assert blocks_rel(p, q).max().item() <= F32_TOL, step
            for sname, signed in FP8_STATES.items():
                if sname in copt.values.get(q, {}):
                    assert gopt.state[p][sname].dtype == copt.dtypes[sname]
                    _compare_codes(gopt.state[p], sname, copt.values[q][sname], signed, stats=stats, expand_min=emin)
                    assert np.all(gopt.state[p][f"expand_{sname}"].cpu().numpy() * emin % 1 == 0)
        print(f"{first}/{second} expand_min {emin} step {step + 1}: worst code-mismatch "
              f"{max(s['code_mismatch'] for _, s in stats):.2e}")


@pytest.mark.parametrize("eps", [1e-8, 1e-20], ids=["hardware-root", "exact-root"])
def test_fp8_adamw_update_forms_against_oracle(eps):
    """The FP8-state AdamW's two forms of the parameter update: the hardware's
    1-ulp square root and reciprocal (taken where eps sqrt(1 - beta2^t) >=
    2^-37, so with the default eps) and the correctly rounded ones (a tiny
    eps).  fp32 parameters, three steps of the toy's AdamW tensors against the
    oracle at the fp32 weights bar, codes as in the other tests."""
    w, draws = _workload_params("toy", None, 256)
    gm, ga = _params(draws, torch.float32)
    cm, ca = _params(draws, torch.float32)
    gopt = CoatStateMonarchMuon(gm, ga, lr=0.02, momentum=0.95, adamw_eps=eps, qargs=QuantizationConfig(),
                                ns_dtype=None)
    copt = ReferenceCoatStateMonarchMuon(cm, ca, lr=0.02, momentum=0.95, adamw_eps=eps, variant="pretrain")
    copt.keep_values = True
    for step in range(3):
        if step:
            _sync(gm + ga, gopt, cm + ca, copt)
        copt.step()
        gopt.step()
        torch.cuda.synchronize()
        stats, worst = [], 0.0
        for p, q in zip(gm + ga, cm + ca):
            e = blocks_rel(p, q).max().item()
            worst = max(worst, e)
            assert e <= F32_TOL, (step, e)
            for sname, signed in FP8_STATES.items():
                if sname in copt.values.get(q, {}):
                    _compare_codes(gopt.state[p], sname, copt.values[q][sname], signed, stats=stats)
        print(f"AdamW eps {eps:g} step {step + 1}: worst weight error {worst:.3e} (bar {F32_TOL})")


@pytest.mark.parametrize("variant,dtype", [("pretrain", torch.float32), ("membench", torch.bfloat16)])
def test_fp8_states_with_groups_straddling_blocks_against_oracle(variant, dtype):
    """Monarch factors whose blocks hold a number of elements that is not a
    multiple of 128 (a 129-column tensor as in ``test_coat_state_muon.py:27``):
    the reference quantizes each state as one flat tensor, so groups straddle
    blocks and the last one is short (``coat_state_muon.py:27-28,53-58``).
    Three steps against the oracle, beside factors whose blocks do align."""
    g = torch.Generator().manual_seed(33)
    shapes = [((2, 129, 100), True), ((3, 100, 129), True), ((2, 64, 64), True), ((1, 40, 33), True),
              ((2, 129, 100), True), ((1000, 129), False), ((77,), False)]
    draws = [(None, m, torch.randn(s, generator=g) * 0.02, torch.randn(s, generator=g) * 1e-3, None)
             for s, m in shapes]
    gm, ga = _params(draws, dtype)
    cm, ca = _params(draws, dtype)
    ns = None if variant == "pretrain" else torch.bfloat16
    gopt = CoatStateMonarchMuon(gm, ga, lr=0.02, momentum=0.95, qargs=QuantizationConfig(), ns_dtype=ns)
    copt = ReferenceCoatStateMonarchMuon(cm, ca, lr=0.02, momentum=0.95, variant=variant)
    copt.keep_values = True
    tol = _weights_bar(dtype, ns)
    gen = torch.Generator().manual_seed(34)
    for step in range(3):
        if step:
            for p, q in zip(gm + ga, cm + ca):   # new gradients each step
                nxt = (torch.randn(p.shape, generator=gen) * 1e-3).to(dtype)
                p.grad = nxt.to(DEV)
                q.grad = nxt.to(DEV)
            _sync(gm + ga, gopt, cm + ca, copt)
        copt.step()
        gopt.step()
        torch.cuda.synchronize()
        stats = []
        for p, q in zip(gm + ga, cm + ca):
            e = blocks_rel(p, q).max().item()
            assert e <= tol, (step, tuple(p.shape), e)
            for sname, signed in FP8_STATES.items():
                if sname in copt.values.get(q, {}):
                    st = gopt.state[p]
                    assert st[sname].dtype == torch.float8_e4m3fn and st[sname].shape == p.shape
                    assert st[f"scale_{sname}"].numel() == (p.numel() + 127) // 128
                    _compare_codes(st, sname, copt.values[q][sname], signed, stats=stats)
        print(f"{variant} straddling groups step {step + 1}: worst code-mismatch "
              f"{max(s['code_mismatch'] for _, s in stats):.2e}")
