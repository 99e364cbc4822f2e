"""numpy restatement of the FP8 optimizer-state codec -- test infrastructure.

Restates ``pretrain/src/models/monarch/coat_state_muon.py``:
``_quantize_kernel`` (``:46-91``) and ``_dequantize_kernel`` (``:22-43``), with
the constants of ``third_party/coat/utils/_fp8_quantization_config.py:20-26``
(group 128, E4M3, expand_min 16) and the other format the reference maps,
E5M2 (``coat_state_muon.py:17``; ``fp8_max`` = ``torch.finfo(dtype).max``,
``:113``).  Each group of 128 consecutive elements of the flattened tensor
(the last group may be short) carries three fp32 values: ``scale``, ``expand``
and ``sqrt_minmax``.

All arithmetic is float32 with correctly rounded operations (numpy float32),
``pow``/``log2`` from the C library.  The reference's Triton kernels use
approximate division/sqrt and CUDA libdevice ``pow``; bit equality with them
is not claimed.  Pinning: ``tests/test_oracle.py`` checks the round-trip error
bound of each format, the constant-group and zero-group special cases, the
exact halving invariant of ``test_coat_state_muon.py:40-51`` and both
encoders against torch's ``float8_e4m3fn`` / ``float8_e5m2`` casts.
"""
from __future__ import annotations

import numpy as np

GROUP = 128          # coat_state_muon.py:16
FP8_MAX = 448.0      # torch.finfo(float8_e4m3fn).max, coat_state_muon.py:113
E5M2_MAX = 57344.0   # torch.finfo(float8_e5m2).max
EXPAND_MIN = 16      # _fp8_quantization_config.py:26
QUANT_EPS = np.float32(1e-30)
F32 = np.float32


# (mantissa bits, exponent bias, largest finite value) of the two OCP formats
FORMATS = {"E4M3": (3, 7, FP8_MAX), "E5M2": (2, 15, E5M2_MAX)}


def fp8_encode(x: np.ndarray, fmt: str = "E4M3") -> np.ndarray:
    """fp32 -> OCP e4m3fn / e5m2 byte, round-to-nearest-even, saturating to
    +-max (the codec's values never exceed it by more than a rounding).

    Pure integer restatement of IEEE rounding (no library cast), so it can pin
    the HIP encoder bit for bit.  32-bit integer arithmetic throughout; the
    subnormal branch scales by a power of two in float32, which is exact."""
    mbits, bias, fmax = FORMATS[fmt]
    x = np.asarray(x, dtype=np.float32)
    sign = ((x.view(np.uint32) >> 31).astype(np.uint8)) << 7
    a = np.abs(x)
    nan = np.isnan(a)
    a = np.where(nan, np.float32(0), np.minimum(a, np.float32(fmax))).astype(np.float32)
    ab = a.view(np.int32)
    exp = (ab >> 23) - 127
    # normal: exponent 1 - bias .. , mbits mantissa bits; round the 24-bit
    # significand to mbits + 1 bits, ties to even
    shift = 23 - mbits
    m_full = (ab & 0x7FFFFF) | 0x800000
    q = m_full >> shift
    rem = m_full & ((1 << shift) - 1)
    half = 1 << (shift - 1)
    q = q + ((rem > half) | ((rem == half) & ((q & 1) == 1))).astype(np.int32)
    e_n = exp + bias
    carry = q >= (2 << mbits)
    q = np.where(carry, q >> 1, q)
    e_n = np.where(carry, e_n + 1, e_n)
    code_n = (e_n << mbits) | (q & ((1 << mbits) - 1))
    # subnormal: value = k * 2^(1 - bias - mbits), k = 0 .. 2^mbits - 1 (2^mbits
    # rounds up to the smallest normal)
    sub_scale = np.float32(2.0 ** (bias - 1 + mbits))
    # exact (a power-of-two scaling); values of the normal branch are capped
    # first, so the integer cast below stays in range
    scaled = np.minimum(a, np.float32(2.0 ** (1 - bias))) * sub_scale
    k = np.floor(scaled)
    frac = scaled - k                                 # exact: k and scaled share the binade
    k = k + ((frac > 0.5) | ((frac == 0.5) & (np.mod(k, 2) == 1)))
    code_s = k.astype(np.int32)                       # k == 2^mbits -> the smallest normal's code, correct
    code = np.where(exp >= 1 - bias, code_n, code_s)
    code = np.where(a == 0, 0, code)
    out = code.astype(np.uint8) | sign
    out = np.where(nan, np.uint8(0x7F) | sign, out)
    return out.astype(np.uint8)


def fp8_decode(code: np.ndarray, fmt: str = "E4M3") -> np.ndarray:
    """OCP e4m3fn / e5m2 byte -> fp32 (exact)."""
    mbits, bias, _ = FORMATS[fmt]
    c = np.asarray(code, dtype=np.uint8).astype(np.int64)
    sign = np.where(c & 0x80, -1.0, 1.0)
    e = (c >> mbits) & ((0x80 >> mbits) - 1)
    m = c & ((1 << mbits) - 1)
    val = np.where(e == 0, m * 2.0 ** (1 - bias - mbits), (1.0 + m / 2.0 ** mbits) * np.exp2(e - float(bias)))
    if fmt == "E4M3":
        val = np.where((c & 0x7F) == 0x7F, np.nan, val)
    else:
        emax = (0x80 >> mbits) - 1
        val = np.where(e == emax, np.where(m == 0, np.inf, np.nan), val)
    return (sign * val).astype(np.float32)


def e4m3_encode(x: np.ndarray) -> np.ndarray:
    return fp8_encode(x, "E4M3")


def e4m3_decode(code: np.ndarray) -> np.ndarray:
    return fp8_decode(code, "E4M3")


def _groups(flat: np.ndarray):
    n = flat.size
    ngroups = (n + GROUP - 1) // GROUP
    padded = np.zeros(ngroups * GROUP, dtype=np.float32)
    padded[:n] = flat
    mask = np.zeros(ngroups * GROUP, dtype=bool)
    mask[:n] = True
    return padded.reshape(ngroups, GROUP), mask.reshape(ngroups, GROUP), n


def quantize(value: np.ndarray, signed: bool, fmt: str = "E4M3", expand_min: float = EXPAND_MIN):
    """Restates ``_quantize_kernel`` (``coat_state_muon.py:46-91``) with
    ``fp8_max`` the format's largest value (``:113``).

    Returns ``(codes uint8 [numel], scale f32 [G], expand f32 [G],
    sqrt_minmax f32 [G])``."""
    fp8_max = FORMATS[fmt][2]
    flat = np.asarray(value, dtype=np.float32).reshape(-1)
    m, mask, n = _groups(flat)
    with np.errstate(divide="ignore", invalid="ignore", over="ignore"):
        abs_m = np.abs(m)
        valid = mask & (abs_m > 0)
        absmax = np.max(np.where(mask, abs_m, F32(0)), axis=1)
        absmin = np.min(np.where(valid, abs_m, F32(3.4028235e38)), axis=1)
        nonzero = valid.sum(axis=1)
        absmax = np.maximum(absmax, QUANT_EPS)
        absmin = np.where(nonzero > 0, np.maximum(absmin, QUANT_EPS), QUANT_EPS).astype(F32)
        ratio = (absmax / absmin).astype(F32)
        ratio = np.maximum(ratio, F32(1.0) + QUANT_EPS)          # 1 + 1e-30 == 1 in f32
        ratio_upper = F32(fp8_max) * F32(fp8_max) / F32(2.0)
        log_ratio = np.log2(ratio).astype(F32)
        safe_log = np.where(log_ratio > QUANT_EPS, log_ratio, F32(1.0)).astype(F32)
        em = F32(expand_min)
        raw_expand = (np.floor((np.log2(ratio_upper).astype(F32) / safe_log) * em) / em).astype(F32)
        expand = np.where(ratio <= F32(1.0) + QUANT_EPS, F32(1.0),
                          np.maximum(raw_expand, F32(1.0) / em)).astype(F32)
        sqrt_minmax = (np.sqrt(absmax) * np.sqrt(absmin)).astype(F32)
        sqrt_minmax = np.maximum(sqrt_minmax, QUANT_EPS)
        norm_base = np.maximum(abs_m / sqrt_minmax[:, None], QUANT_EPS).astype(F32)
        norm_pow = np.power(norm_base, expand[:, None]).astype(F32)
        if signed:
            sgn = np.where(m >= 0, F32(1.0), F32(-1.0))
            normalized = np.where(mask & (abs_m > 0), sgn * norm_pow, F32(0)).astype(F32)
        else:
            normalized = np.where(mask & (abs_m > 0), norm_pow, F32(0)).astype(F32)
        scale_base = np.maximum(absmax / sqrt_minmax, QUANT_EPS).astype(F32)
        scale = (np.power(scale_base, expand).astype(F32) / F32(fp8_max)).astype(F32)
        scale = np.maximum(scale, QUANT_EPS)
        q = (normalized / scale[:, None]).astype(F32)
    codes = fp8_encode(q, fmt).reshape(-1)[:n]
    return codes, scale.astype(F32), expand.astype(F32), sqrt_minmax.astype(F32)


def dequantize(codes: np.ndarray, scale, expand, sqrt_minmax, signed: bool, fmt: str = "E4M3") -> np.ndarray:
    """Restates ``_dequantize_kernel`` (``coat_state_muon.py:22-43``)."""
    flat = fp8_decode(np.asarray(codes).reshape(-1), fmt)
    raw, mask, n = _groups(flat)
    s = np.asarray(scale, dtype=F32)[:, None]
    with np.errstate(divide="ignore", invalid="ignore", over="ignore"):
        ex = np.maximum(np.asarray(expand, dtype=F32), QUANT_EPS)[:, None]
        smm = np.maximum(np.asarray(sqrt_minmax, dtype=F32), QUANT_EPS)[:, None]
        inv = (F32(1.0) / ex).astype(F32)
        if signed:
            scaled = (raw * s).astype(F32)
            absolute = np.abs(scaled)
            sgn = np.where(scaled >= 0, F32(1.0), F32(-1.0))
            power = np.power(np.maximum(absolute, QUANT_EPS), inv).astype(F32)
            value = np.where(absolute > 0, (sgn * power).astype(F32) * smm, F32(0)).astype(F32)
        else:
            scaled = np.maximum((raw * s).astype(F32), F32(0))
            power = np.power(np.maximum(scaled, QUANT_EPS), inv).astype(F32)
            value = np.where(scaled > 0, power * smm, F32(0)).astype(F32)
    return value.reshape(-1)[:n]
