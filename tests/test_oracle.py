"""Pins the CPU oracle (oracle/) before it is trusted as the parity checker.

Each check is chosen so a plausible restatement mistake (dropped term, wrong
sign, transposed operand, wrong rounding point) fails it.
"""
import math

import numpy as np
import pytest
import torch

from golden_inputs import CASES, input_checksum, make_case
from oracle import codec, shapes
from oracle.step import NS_COEFFS, ReferenceMonarchMuon, group_blocks, newton_schulz_batched
from oracle.truth import known_answer, ns_fp64, quintic_scalar, rel_fro

GOLDEN = __import__("pathlib").Path(__file__).resolve().parent / "golden"


# ---------------------------------------------------------------- golden vectors
@pytest.mark.parametrize("case", CASES, ids=[c["name"] for c in CASES])
def test_oracle_matches_reference_golden(case):
    gold = torch.load(GOLDEN / f"{case['name']}.pt", weights_only=True)
    assert gold["inputs_sha"] == input_checksum(case), "seeded input generator drifted"
    muon, adamw, bufs = make_case(case)
    opt = ReferenceMonarchMuon(muon, adamw, lr=case["lr"], momentum=0.95, variant=case["variant"])
    if bufs is not None:
        for p, b in zip(muon, bufs):
            opt.state[p]["momentum_buffer"] = b
    for _ in range(case["steps"]):
        opt.step()
    tol = dict(rtol=1e-6, atol=1e-9)
    for p, q in zip(muon, gold["muon_params"]):
        torch.testing.assert_close(p.detach(), q, **tol)
    for p, q in zip(muon, gold["momentum"]):
        torch.testing.assert_close(opt.state[p]["momentum_buffer"], q, **tol)
    for p, q in zip(adamw, gold["adamw_params"]):
        torch.testing.assert_close(p.detach(), q, **tol)
    for p, q, r in zip(adamw, gold["exp_avg"], gold["exp_avg_sq"]):
        torch.testing.assert_close(opt.state[p]["exp_avg"], q, **tol)
        torch.testing.assert_close(opt.state[p]["exp_avg_sq"], r, **tol)
    torch.testing.assert_close(newton_schulz_batched(gold["ns_input"]), gold["ns_output"], rtol=0, atol=0)


# ---------------------------------------------------------------- Newton-Schulz
def _svd_case(r, c, seed):
    g = torch.Generator().manual_seed(seed)
    k = min(r, c)
    u, _ = torch.linalg.qr(torch.randn(r, k, generator=g, dtype=torch.float64))
    v, _ = torch.linalg.qr(torch.randn(c, k, generator=g, dtype=torch.float64))
    s = torch.rand(k, generator=g, dtype=torch.float64) * 2 + 0.01
    return u, s, v, (u * s) @ v.T


@pytest.mark.parametrize("r,c", [(24, 24), (40, 16), (16, 40)])
def test_ns_known_answer_svd(r, c):
    u, s, v, x = _svd_case(r, c, 3)
    out = newton_schulz_batched(x[None])[0]
    ref = known_answer(u, s, v)
    assert rel_fro(out, ref) < 1e-12
    # the scalar quintic is what acts on each singular value
    sv = torch.linalg.svdvals(out).sort().values
    phi = torch.from_numpy(np.sort(quintic_scalar((s / (s.norm() + 1e-7)).numpy())))
    torch.testing.assert_close(sv, phi, rtol=1e-10, atol=1e-12)


def test_ns_diagonal_exact():
    d = torch.diag(torch.tensor([3.0, 1.0, 0.5, 0.25], dtype=torch.float64))
    out = newton_schulz_batched(d[None])[0]
    expect = quintic_scalar((torch.diagonal(d) / (torch.diagonal(d).norm() + 1e-7)).numpy())
    torch.testing.assert_close(torch.diagonal(out), torch.from_numpy(expect))
    assert torch.count_nonzero(out - torch.diag(torch.diagonal(out))) == 0


def test_ns_invariants():
    g = torch.Generator().manual_seed(5)
    x = torch.randn(20, 33, generator=g, dtype=torch.float64)
    q, _ = torch.linalg.qr(torch.randn(20, 20, generator=g, dtype=torch.float64))
    rr, _ = torch.linalg.qr(torch.randn(33, 33, generator=g, dtype=torch.float64))
    f = lambda t: newton_schulz_batched(t[None])[0]
    torch.testing.assert_close(f(q @ x @ rr), q @ f(x) @ rr, rtol=1e-9, atol=1e-10)
    torch.testing.assert_close(f(x.T), f(x).T, rtol=1e-12, atol=1e-13)
    # equal up to the 1e-7 in the normaliser, amplified by the quintic slope (~3.4445^5)
    torch.testing.assert_close(f(7.5 * x), f(x), rtol=1e-4, atol=1e-7)
    assert torch.count_nonzero(f(torch.zeros(5, 9, dtype=torch.float64))) == 0


def test_ns_matches_fp64_three_product_form_in_fp64():
    g = torch.Generator().manual_seed(6)
    x = torch.randn(3, 24, 40, generator=g, dtype=torch.float64)
    assert rel_fro(newton_schulz_batched(x), ns_fp64(x)).max() < 1e-12


def test_ns_coefficients_are_the_reference_quintic():
    # phi(x) = a x + b x^3 + c x^5 with a + b + c = 0.7010 (not a fixed point at 1 on purpose)
    a, b, c = NS_COEFFS
    assert (a, b, c) == (3.4445, -4.7750, 2.0315)
    assert quintic_scalar(np.array([0.0]))[0] == 0.0


# ---------------------------------------------------------------- momentum / apply
def test_momentum_and_apply_brute_force_fp64():
    g = torch.Generator().manual_seed(7)
    w = (torch.randn(2, 8, 12, generator=g) * 0.02)
    gr = torch.randn(2, 8, 12, generator=g) * 1e-3
    buf = torch.randn(2, 8, 12, generator=g) * 1e-3
    p = w.clone().requires_grad_(True)
    p.grad = gr.clone()
    opt = ReferenceMonarchMuon([p], [], lr=0.05, momentum=0.9, variant="pretrain")
    opt.state[p]["momentum_buffer"] = buf.clone()
    opt.step()
    # two fp32 roundings (mul_ then add_), no fused multiply-add
    nb32 = (buf.numpy() * np.float32(0.9)).astype(np.float32) + gr.numpy()
    np.testing.assert_array_equal(opt.state[p]["momentum_buffer"].numpy(), nb32)
    nb = 0.9 * buf.double() + gr.double()
    torch.testing.assert_close(opt.state[p]["momentum_buffer"].double(), nb, rtol=0, atol=1e-9)
    upd = ns_fp64(nb)
    expect = w.double() - 0.05 * math.sqrt(8 / 12) * upd
    torch.testing.assert_close(p.detach().double(), expect, rtol=1e-5, atol=1e-7)


def test_grad_none_is_skipped_and_zero_grad_gives_zero_update():
    p = torch.randn(1, 8, 8).requires_grad_(True)
    q = torch.randn(1, 8, 8).requires_grad_(True)
    q.grad = torch.zeros_like(q)
    p0, q0 = p.detach().clone(), q.detach().clone()
    opt = ReferenceMonarchMuon([p, q], [], variant="membench")
    opt.step()
    assert torch.equal(p.detach(), p0) and "momentum_buffer" not in opt.state[p]
    assert torch.equal(q.detach(), q0)


# ---------------------------------------------------------------- AdamW
@pytest.mark.parametrize("variant", ["membench", "pretrain"])
def test_adamw_matches_torch_adamw(variant):
    g = torch.Generator().manual_seed(8)
    ws = [torch.randn(17, 5, generator=g, dtype=torch.float64), torch.randn(9, generator=g, dtype=torch.float64)]
    a = [w.clone().requires_grad_(True) for w in ws]
    b = [w.clone().requires_grad_(True) for w in ws]
    ours = ReferenceMonarchMuon([], a, lr=1e-2, adamw_betas=(0.9, 0.95), adamw_weight_decay=0.1,
                                adamw_eps=1e-8, variant=variant)
    lib = torch.optim.AdamW(b, lr=1e-2, betas=(0.9, 0.95), weight_decay=0.1, eps=1e-8, foreach=False)
    for step in range(3):
        grads = [torch.randn(w.shape, generator=g, dtype=torch.float64) for w in ws]
        for x, y, gr in zip(a, b, grads):
            x.grad, y.grad = gr.clone(), gr.clone()
        ours.step()
        lib.step()
    for x, y in zip(a, b):
        torch.testing.assert_close(x.detach(), y.detach(), rtol=1e-12, atol=1e-14)


# ---------------------------------------------------------------- grouping / shapes
def test_grouping_first_appearance_order():
    bufs = [torch.zeros(2, 4, 4), torch.zeros(1, 6, 4), torch.zeros(1, 4, 4), torch.zeros(1, 6, 4, dtype=torch.bfloat16)]
    keys = list(group_blocks(bufs, bufs).keys())
    assert [(k[1], k[2], k[3]) for k in keys] == [(torch.float32, 4, 4), (torch.float32, 6, 4), (torch.bfloat16, 6, 4)]
    assert [i for i, _, _ in group_blocks(bufs, bufs)[keys[0]]] == [0, 2]


MEMBENCH_COUNTS = [  # membench/scripts/monarch_benchmark/common.py:13-64
    (12, 1024, 0, 163_603_456), (24, 1536, 0, 423_568_896), (24, 2048, 0, 690_587_648),
    (28, 3072, 0, 1_564_388_352), (32, 4096, 11008, 2_970_882_048)]


@pytest.mark.parametrize("layers,embd,inter,expected", MEMBENCH_COUNTS)
def test_shape_rule_matches_reference_parameter_counts(layers, embd, inter, expected):
    ps = shapes.llama_monarch_params(layers, embd, inter, 4)
    assert sum(math.prod(s) for _, s in ps) == expected


# ---------------------------------------------------------------- FP8 codec
FMTS = {"E4M3": (torch.float8_e4m3fn, 448.0, 0x7E), "E5M2": (torch.float8_e5m2, 57344.0, 0x7B)}


@pytest.mark.parametrize("fmt", list(FMTS))
def test_fp8_encoder_matches_torch_cast(fmt):
    dt, fmax, _ = FMTS[fmt]
    lo = -12 if fmt == "E4M3" else -19
    hi = 9 if fmt == "E4M3" else 16
    x = np.concatenate([np.linspace(-1.03 * fmax, 1.03 * fmax, 20001, dtype=np.float32),
                        np.float32(2.0) ** np.arange(lo, hi, 0.125, dtype=np.float32),
                        -np.float32(2.0) ** np.arange(lo, hi, 0.125, dtype=np.float32),
                        np.array([0.0, -0.0], dtype=np.float32)])
    # every representable value and every midpoint between neighbours (ties to even)
    allv = np.unique(np.abs(torch.arange(256, dtype=torch.uint8).view(dt).float().numpy()))
    allv = allv[np.isfinite(allv)]
    mids = ((allv[1:].astype(np.float64) + allv[:-1]) / 2).astype(np.float32)
    x = np.concatenate([x, allv, -allv, mids, -mids])
    clipped = np.clip(x, -fmax, fmax)
    ours = codec.fp8_encode(x, fmt)
    ref = torch.from_numpy(clipped).to(dt).view(torch.uint8).numpy()
    np.testing.assert_array_equal(ours, ref)
    np.testing.assert_array_equal(codec.fp8_decode(ours, fmt), torch.from_numpy(ref).view(dt).float().numpy())
    codes = np.arange(256, dtype=np.uint8)
    np.testing.assert_array_equal(codec.fp8_decode(codes, fmt),
                                  torch.from_numpy(codes).view(dt).float().numpy())


def _decades(n, seed):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal(n) * np.logspace(-6, 1, n)).astype(np.float32)


@pytest.mark.parametrize("fmt", list(FMTS))
@pytest.mark.parametrize("signed", [True, False])
def test_codec_round_trip_bound(signed, fmt):
    x = _decades(1000 * 129, 9).reshape(1000, 129)      # tail group + 7 decades (test_coat_state_muon.py:27-28)
    if not signed:
        x = x * x
    fmax = FMTS[fmt][1]
    q, sc, ex, smm = codec.quantize(x, signed, fmt)
    y = codec.dequantize(q, sc, ex, smm, signed, fmt).reshape(x.shape)
    # The encoder stores q = fmax (|x|/absmax)^expand; the format keeps q to a
    # relative 2^-(mbits+1) when normal and to an absolute half of its smallest
    # subnormal below.  The decoder raises back to 1/expand, so
    # |y/x - 1| <= 1 - (1 - eq)^(1/expand).
    rel_q, abs_q = (2.0 ** -4, 2.0 ** -10) if fmt == "E4M3" else (2.0 ** -3, 2.0 ** -17)
    xf, yf = x.reshape(-1).astype(np.float64), y.reshape(-1).astype(np.float64)
    groups = np.arange(xf.size) // 128
    amax = np.maximum.reduceat(np.abs(xf), np.arange(0, xf.size, 128))[groups]
    e = ex[groups].astype(np.float64)
    qv = fmax * (np.abs(xf) / amax) ** e
    eq = np.maximum(rel_q, abs_q / np.maximum(qv, 1e-300))
    bound = np.maximum(1 - np.clip(1 - eq, 0, None) ** (1.0 / e), (1 + eq) ** (1.0 / e) - 1) + 1e-5
    rel = np.abs(yf - xf) / np.maximum(np.abs(xf), 1e-300)
    nz = xf != 0
    assert np.all(rel[nz] <= bound[nz])
    assert np.all(yf[~nz] == 0)
    assert np.all(np.sign(y.reshape(-1)) == np.sign(x.reshape(-1)) * (y.reshape(-1) != 0)) or not signed


@pytest.mark.parametrize("fmt", list(FMTS))
def test_codec_special_groups(fmt):
    fmax = FMTS[fmt][1]
    const = np.full(128, 0.37, dtype=np.float32)
    q, sc, ex, smm = codec.quantize(const, True, fmt)
    assert ex[0] == 1.0                                    # ratio 1 -> expand = 1
    np.testing.assert_allclose(codec.dequantize(q, sc, ex, smm, True, fmt), const, rtol=2 ** -3)
    z = np.zeros(300, dtype=np.float32)
    q, sc, ex, smm = codec.quantize(z, True, fmt)
    assert np.all(q == 0) and np.all(codec.dequantize(q, sc, ex, smm, True, fmt) == 0)
    # group of 2 decades: expand = floor(log2(fmax^2/2)/log2(100)*16)/16
    x = np.array([1.0, 100.0] * 64, dtype=np.float32)
    _, _, ex, smm = codec.quantize(x, False, fmt)
    upper = np.float32(fmax) * np.float32(fmax) / np.float32(2)
    assert ex[0] == np.floor(np.log2(upper) / np.log2(np.float32(100.0)) * 16) / 16
    assert smm[0] == np.float32(10.0)
    # both signed zeros store +0's code (the masked 0.0 of coat_state_muon.py:79)
    v = np.array([1.0, -0.0, 0.0, -0.25] + [0.5] * 124, dtype=np.float32)
    q, *_ = codec.quantize(v, True, fmt)
    assert q[1] == 0 and q[2] == 0 and q[3] >> 7 == 1


@pytest.mark.parametrize("emin", [16, 8, 4, 1, 32])
def test_codec_expand_min(emin):
    # expand = floor(log2(448^2/2) / log2(ratio) * emin) / emin, at least 1/emin
    # (coat_state_muon.py:69-71 with the config's expand_min)
    upper = np.float32(448.0) * np.float32(448.0) / np.float32(2)
    for ratio in (100.0, 1e4, 3.0, 1e30):
        x = np.array([1.0, ratio] * 64, dtype=np.float32)
        _, _, ex, _ = codec.quantize(x, True, "E4M3", emin)
        r = np.float32(ratio)
        raw = np.float32(np.floor(np.float32(np.log2(upper) / np.log2(r)) * np.float32(emin)) / np.float32(emin))
        assert ex[0] == max(raw, np.float32(1.0) / np.float32(emin)), (emin, ratio, ex[0])
        assert ex[0] * emin == np.floor(ex[0] * emin)                     # a multiple of 1/emin
    # the floor at 1/emin acts for a group spanning more than 16.6 * emin octaves
    x = np.array([1e-30, 1e30] * 64, dtype=np.float32)
    assert codec.quantize(x, True, "E4M3", 1)[2][0] == 1.0


@pytest.mark.parametrize("fmt", list(FMTS))
def test_codec_group_max_encodes_to_fp8_max(fmt):
    # q = sign * (|x|/smm)^e / ((absmax/smm)^e / fmax): the largest |value| of every
    # group lands on +-fmax, which pins scale against expand and smm
    _, fmax, maxcode = FMTS[fmt]
    x = _decades(1000 * 129, 10)
    for signed in (True, False):
        v = x if signed else x * x
        q, sc, ex, smm = codec.quantize(v, signed, fmt)
        g = (v.size + 127) // 128
        pad = np.zeros(g * 128, dtype=np.float32)
        pad[:v.size] = v
        top = np.argmax(np.abs(pad.reshape(g, 128)), axis=1) + np.arange(g) * 128
        assert np.all(q[top] & 0x7F == maxcode)
        assert np.all((q[top] >> 7) == (pad[top] < 0))
        # and it decodes back to that value within the format + power rounding
        d = codec.dequantize(q, sc, ex, smm, signed, fmt)
        np.testing.assert_allclose(d[top], pad[top], rtol=1e-5)


@pytest.mark.parametrize("fmt", list(FMTS))
def test_codec_power_of_four_homogeneity(fmt):
    # scaling a group by 4 (or 1/4) scales absmax, absmin and sqrt(absmax)*sqrt(absmin)
    # exactly (sqrt(4a) = 2 sqrt(a) in IEEE arithmetic), so codes, scale and expand
    # are unchanged and sqrt_minmax is scaled by exactly 4; the decoder is linear in it
    x = _decades(1000 * 129, 11)
    for signed in (True, False):
        v = x if signed else x * x
        q, sc, ex, smm = codec.quantize(v, signed, fmt)
        for f in (np.float32(4.0), np.float32(0.25)):
            q2, sc2, ex2, smm2 = codec.quantize(v * f, signed, fmt)
            np.testing.assert_array_equal(q2, q)
            np.testing.assert_array_equal(sc2, sc)
            np.testing.assert_array_equal(ex2, ex)
            np.testing.assert_array_equal(smm2, smm * f)
        d = codec.dequantize(q, sc, ex, smm, signed, fmt)
        np.testing.assert_array_equal(codec.dequantize(q, sc, ex, smm * np.float32(4), signed, fmt),
                                      d * np.float32(4))


@pytest.mark.parametrize("fmt", list(FMTS))
def test_codec_halving_after_dequantize(fmt):
    # the pattern of test_coat_state_muon.py:40-51 (dequantize, halve exactly,
    # requantize): the halved group keeps its codes and expansion, and its
    # sqrt_minmax and scale move by at most an ulp or two (sqrt(a/2) is not
    # exactly sqrt(a)/sqrt(2))
    x = _decades(1000 * 129, 12)
    for signed in (True, False):
        v = x if signed else x * x
        d = codec.dequantize(*codec.quantize(v, signed, fmt), signed, fmt)
        full = codec.quantize(d, signed, fmt)
        half = codec.quantize(d * np.float32(0.5), signed, fmt)
        np.testing.assert_array_equal(half[0], full[0])
        np.testing.assert_array_equal(half[2], full[2])
        np.testing.assert_allclose(half[3], full[3] * np.float32(0.5), rtol=3e-7, atol=0)
        # scale = (absmax/smm)^expand / fmax: an ulp of smm plus the division's
        # rounding move the base by up to ~1.5 ulps, which the power multiplies
        # by expand; pow and the division by fmax add an ulp each
        rel = np.abs(half[1].astype(np.float64) / full[1] - 1)
        assert np.all(rel <= (2 * full[2].astype(np.float64) + 3) * 2.0 ** -23)


# ---------------------------------------------------------------- FP8-state wrapper (coat_state_muon.py:117-139)
def _coat_inputs(dtype, seed=20):
    g = torch.Generator().manual_seed(seed)
    shapes = [(2, 64, 64), (1, 128, 64), (1, 64, 128)]
    muon = []
    for s in shapes:
        p = (torch.randn(s, generator=g) * 0.02).to(dtype).requires_grad_(True)
        p.grad = (torch.randn(s, generator=g) * 1e-3).to(dtype)
        muon.append(p)
    a = (torch.randn(100, 64, generator=g) * 0.02).to(dtype).requires_grad_(True)
    a.grad = (torch.randn(100, 64, generator=g) * 1e-3).to(dtype)
    return muon, [a]


def _clone(ps):
    out = []
    for p in ps:
        q = p.detach().clone().requires_grad_(True)
        q.grad = p.grad.clone()
        out.append(q)
    return out


COAT_CASES = [("pretrain", torch.float32), ("pretrain", torch.bfloat16), ("membench", torch.bfloat16)]


@pytest.mark.parametrize("variant,dtype", COAT_CASES)
def test_coat_oracle_first_step_is_unwrapped_step_then_quantize(variant, dtype):
    from oracle.step import FP8_STATES, ReferenceCoatStateMonarchMuon
    muon, adamw = _coat_inputs(dtype)
    m2, a2 = _clone(muon), _clone(adamw)
    wrapped = ReferenceCoatStateMonarchMuon(muon, adamw, lr=0.02, variant=variant)
    plain = ReferenceMonarchMuon(m2, a2, lr=0.02, variant=variant)
    wrapped.step()
    plain.step()
    for p, q in zip(muon + adamw, m2 + a2):
        assert torch.equal(p, q)                     # quantization happens after the step
        for name, signed in FP8_STATES.items():
            if name not in plain.state[q]:
                continue
            value = plain.state[q][name]
            assert value.dtype == dtype              # created by zeros_like(param)
            codes, sc, ex, smm = codec.quantize(value.float().numpy(), signed)
            st = wrapped.state[p]
            assert st[name].dtype == torch.float8_e4m3fn
            np.testing.assert_array_equal(st[name].view(torch.uint8).numpy().reshape(-1), codes)
            for key, ref in zip(("scale", "expand", "sqrt_minmax"), (sc, ex, smm)):
                assert st[f"{key}_{name}"].dtype == torch.float32
                np.testing.assert_array_equal(st[f"{key}_{name}"].numpy(), ref)


@pytest.mark.parametrize("variant,dtype", COAT_CASES)
def test_coat_oracle_later_step_runs_on_fp32_dequantized_states(variant, dtype):
    from oracle.step import ReferenceCoatStateMonarchMuon
    muon, adamw = _coat_inputs(dtype, seed=21)
    wrapped = ReferenceCoatStateMonarchMuon(muon, adamw, lr=0.02, variant=variant)
    wrapped.step()
    # an unwrapped copy started from the decoded states (decoded here, with the
    # signedness spelled out per state) must take the same second step
    m2, a2 = _clone(muon), _clone(adamw)
    plain = ReferenceMonarchMuon(m2, a2, lr=0.02, variant=variant)
    decode = lambda st, n, s: torch.from_numpy(codec.dequantize(
        st[n].view(torch.uint8).numpy().reshape(-1), st[f"scale_{n}"].numpy(), st[f"expand_{n}"].numpy(),
        st[f"sqrt_minmax_{n}"].numpy(), s)).reshape(st[n].shape)
    for p, q in zip(muon, m2):
        plain.state[q]["momentum_buffer"] = decode(wrapped.state[p], "momentum_buffer", True)
    for p, q in zip(adamw, a2):
        st = wrapped.state[p]
        plain.state[q].update(step=st["step"], exp_avg=decode(st, "exp_avg", True),
                              exp_avg_sq=decode(st, "exp_avg_sq", False))
    wrapped.step()
    plain.step()
    for p, q in zip(muon + adamw, m2 + a2):
        assert torch.equal(p, q)
    for p, q in zip(muon, m2):
        assert plain.state[q]["momentum_buffer"].dtype == torch.float32
        codes = codec.quantize(plain.state[q]["momentum_buffer"].numpy(), True)[0]
        np.testing.assert_array_equal(wrapped.state[p]["momentum_buffer"].view(torch.uint8).numpy().reshape(-1),
                                      codes)


def test_coat_oracle_halving_pattern():
    # test_coat_state_muon.py:40-51 applied to the wrapper's AdamW states: with
    # betas (0.5, 0.5), lr 0 and zero gradients the step halves both moments
    # exactly, so the stored states are the quantized halves of the decoded ones
    from oracle.step import ReferenceCoatStateMonarchMuon, dequantize_state
    _, adamw = _coat_inputs(torch.float32, seed=22)
    opt = ReferenceCoatStateMonarchMuon([], adamw, lr=0.02, adamw_weight_decay=0.0, variant="pretrain")
    opt.step()
    p = adamw[0]
    before = {n: dequantize_state(opt.state[p], n, s) for n, s in (("exp_avg", True), ("exp_avg_sq", False))}
    for group in opt.param_groups:
        group["betas"] = (0.5, 0.5)
        group["lr"] = 0.0
    p.grad.zero_()
    w = p.detach().clone()
    opt.step()
    assert torch.equal(p, w)
    for name, signed in (("exp_avg", True), ("exp_avg_sq", False)):
        codes, sc, ex, smm = codec.quantize((before[name] * 0.5).numpy(), signed)
        st = opt.state[p]
        np.testing.assert_array_equal(st[name].view(torch.uint8).numpy().reshape(-1), codes)
        np.testing.assert_array_equal(st[f"scale_{name}"].numpy(), sc)
        np.testing.assert_array_equal(st[f"expand_{name}"].numpy(), ex)
        np.testing.assert_array_equal(st[f"sqrt_minmax_{name}"].numpy(), smm)
