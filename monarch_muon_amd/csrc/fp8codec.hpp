// FP8 (OCP e4m3fn, group-128, dynamic range expansion) optimizer-state codec.
//
// Device restatement of the codec of coat_state_muon.py:22-91 (itself the
// first/second-order half of COAT's AdamW expand kernel).  Each group of 128
// consecutive elements carries fp32 scale, expand and sqrt_minmax.  A group is
// held by a few lanes of a wave, a run of consecutive elements per lane.
#pragma once

#include "common.hpp"

namespace mmuon {

constexpr float FP8_MAX = 448.0f;
constexpr float QEPS = 1e-30f;
constexpr float LOG2_QEPS = -99.657842847f;  // log2(QEPS)
constexpr float EXPAND_MIN = 16.0f;

// e4m3fn byte -> fp32 (exact).
__device__ __forceinline__ float e4m3_decode(uint32_t c) {
  const uint32_t e = (c >> 3) & 0xfu, m = c & 7u;
  float v;
  if ((c & 0x7fu) == 0x7fu) v = __uint_as_float(0x7fc00000u);
  else if (e == 0u) v = float(m) * (1.0f / 512.0f);
  else v = __uint_as_float(((e + 120u) << 23) | (m << 20));
  return (c & 0x80u) ? -v : v;
}

struct Fp8Meta {
  float scale, expand, sqrt_minmax;
};

// x^y for a positive normal x, as 2^(y log2 x) with the hardware base-2
// logarithm and exponential (v_log_f32, v_exp_f32).  Rounding the product
// y log2 x adds a relative error of about |y log2 x| * 2^-24 to the result; the
// codec's per-element powers have |y log2 x| below ~20 for any group whose
// values are not denormal-scale, so the result stays within ~1e-6 relative.
__device__ __forceinline__ float pow_pos(float x, float y) {
  return __builtin_amdgcn_exp2f(y * __builtin_amdgcn_logf(x));
}

// Per-group dequantization constants: scale, 1/expand, sqrt_minmax (clamped
// as coat_state_muon.py:34-36 clamps them).
struct Fp8Dq {
  float scale, inv_expand, smm;
};
__device__ __forceinline__ Fp8Dq fp8_dq(const Fp8Meta& md) {
  return Fp8Dq{md.scale, 1.0f / fmaxf(md.expand, QEPS), fmaxf(md.sqrt_minmax, QEPS)};
}

// coat_state_muon.py:22-43 for one element.
__device__ __forceinline__ float fp8_dequant(uint32_t code, const Fp8Dq& d, bool sgn) {
  const float raw = e4m3_decode(code);
  if (sgn) {
    const float scaled = raw * d.scale;
    const float absolute = fabsf(scaled);
    const float s = scaled >= 0.f ? 1.f : -1.f;
    const float power = pow_pos(fmaxf(absolute, QEPS), d.inv_expand);
    return absolute > 0.f ? (s * power) * d.smm : 0.f;
  }
  const float scaled = fmaxf(raw * d.scale, 0.f);
  const float power = pow_pos(fmaxf(scaled, QEPS), d.inv_expand);
  return scaled > 0.f ? power * d.smm : 0.f;
}
__device__ __forceinline__ float fp8_dequant(uint32_t code, const Fp8Meta& md, bool sgn) {
  return fp8_dequant(code, fp8_dq(md), sgn);
}

// ---------------------------------------------------------------------------
// A group of 128 is held by 128/E lanes, E consecutive elements per lane (E a
// multiple of 16: whole 16-byte code accesses).  gfx950's v_cvt_f32_fp8 /
// v_cvt_pk_fp8_f32 convert OCP e4m3fn with round-to-nearest-even (the rounding
// torch's float8_e4m3fn cast uses); the encoder's inputs are clamped to +-448
// first, as the codec saturates.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void e4m3_decode4(uint32_t c, float* v) {
  v[0] = __builtin_amdgcn_cvt_f32_fp8(int(c), 0);
  v[1] = __builtin_amdgcn_cvt_f32_fp8(int(c), 1);
  v[2] = __builtin_amdgcn_cvt_f32_fp8(int(c), 2);
  v[3] = __builtin_amdgcn_cvt_f32_fp8(int(c), 3);
}
// values already clamped to [-448, 448]
__device__ __forceinline__ uint32_t e4m3_encode4(const float* v) {
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(v[0], v[1], 0, false);
  w = __builtin_amdgcn_cvt_pk_fp8_f32(v[2], v[3], w, true);
  return uint32_t(w);
}

// Cross-lane max / min over the 128/E lanes of a group (every lane of the
// group active): swap neighbours, swap pairs (, mirror the halves of 8).
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xf, 0xf, false));
}
template <int LANES>
__device__ __forceinline__ float group_max(float v) {
  static_assert(LANES == 4 || LANES == 8, "groups of 4 or 8 lanes");
  v = fmaxf(v, dpp_f<0xb1>(v));                      // quad_perm [1,0,3,2]
  v = fmaxf(v, dpp_f<0x4e>(v));                      // quad_perm [2,3,0,1]
  if constexpr (LANES == 8) v = fmaxf(v, dpp_f<0x141>(v));  // row_half_mirror
  return v;
}
template <int LANES>
__device__ __forceinline__ float group_min(float v) {
  static_assert(LANES == 4 || LANES == 8, "groups of 4 or 8 lanes");
  v = fminf(v, dpp_f<0xb1>(v));
  v = fminf(v, dpp_f<0x4e>(v));
  if constexpr (LANES == 8) v = fminf(v, dpp_f<0x141>(v));
  return v;
}

// coat_state_muon.py:22-43 for this lane's E elements of one group.
template <int E>
__device__ __forceinline__ void fp8_dequant_lane(const uint4 (&codes)[E / 16], const Fp8Dq& d, bool sgn,
                                                 float (&out)[E]) {
  float raw[E];
#pragma unroll
  for (int h = 0; h < E / 16; ++h) {
    e4m3_decode4(codes[h].x, raw + 16 * h);
    e4m3_decode4(codes[h].y, raw + 16 * h + 4);
    e4m3_decode4(codes[h].z, raw + 16 * h + 8);
    e4m3_decode4(codes[h].w, raw + 16 * h + 12);
  }
#pragma unroll
  for (int k = 0; k < E; ++k) {
    if (sgn) {
      const float scaled = raw[k] * d.scale;
      const float absolute = fabsf(scaled);
      const float power = pow_pos(fmaxf(absolute, QEPS), d.inv_expand);
      out[k] = absolute > 0.f ? copysignf(power, scaled) * d.smm : 0.f;
    } else {
      const float scaled = fmaxf(raw[k] * d.scale, 0.f);
      const float power = pow_pos(fmaxf(scaled, QEPS), d.inv_expand);
      out[k] = scaled > 0.f ? power * d.smm : 0.f;
    }
  }
}

// coat_state_muon.py:46-91 for one group (nvalid: this lane's elements that
// exist).  Returns the group metadata (valid in every lane of the group) and
// this lane's E codes.  Each element's power and its division by scale are one
// exp2 of a log-domain expression, and scale's power uses pow_pos (both visible
// only at e4m3 rounding ties).
template <int E>
__device__ __forceinline__ Fp8Meta fp8_quant_group(const float (&x)[E], int nvalid, bool sgn, uint4 (&codes)[E / 16]) {
  float amax = 0.f, amin = 3.4028235e38f;
#pragma unroll
  for (int k = 0; k < E; ++k) {
    const float a = fabsf(x[k]);
    if (k < nvalid) {
      amax = fmaxf(amax, a);
      if (a > 0.f) amin = fminf(amin, a);
    }
  }
  amax = fmaxf(group_max<128 / E>(amax), QEPS);
  amin = group_min<128 / E>(amin);
  amin = amin < 3.4028235e38f ? fmaxf(amin, QEPS) : QEPS;  // no non-zero value: QEPS
  float ratio = amax / amin;
  ratio = fmaxf(ratio, 1.0f + QEPS);
  const float ratio_upper = FP8_MAX * FP8_MAX / 2.0f;
  const float log_ratio = log2f(ratio);
  const float safe_log = log_ratio > QEPS ? log_ratio : 1.0f;
  const float raw_expand = floorf((log2f(ratio_upper) / safe_log) * EXPAND_MIN) / EXPAND_MIN;
  const float expand = ratio <= 1.0f + QEPS ? 1.0f : fmaxf(raw_expand, 1.0f / EXPAND_MIN);
  const float smm = fmaxf(sqrtf(amax) * sqrtf(amin), QEPS);
  const float scale = fmaxf(pow_pos(fmaxf(amax / smm, QEPS), expand) / FP8_MAX, QEPS);
  // per element, in the log domain: (max(a / smm, QEPS))^expand / scale =
  // 2^(expand * max(log2 a - log2 smm, log2 QEPS) - log2 scale)
  const float lsmm = __builtin_amdgcn_logf(smm), lsc = __builtin_amdgcn_logf(scale);
  float y[E];
#pragma unroll
  for (int k = 0; k < E; ++k) {
    const float a = fabsf(x[k]);
    const float t = fmaxf(__builtin_amdgcn_logf(a) - lsmm, LOG2_QEPS);
    const float np = __builtin_amdgcn_exp2f(fmaf(expand, t, -lsc));
    float nrm = 0.f;
    if (k < nvalid && a > 0.f) nrm = sgn ? copysignf(np, x[k]) : np;
    y[k] = __builtin_amdgcn_fmed3f(nrm, -FP8_MAX, FP8_MAX);
  }
#pragma unroll
  for (int h = 0; h < E / 16; ++h)
    codes[h] = make_uint4(e4m3_encode4(y + 16 * h), e4m3_encode4(y + 16 * h + 4), e4m3_encode4(y + 16 * h + 8),
                          e4m3_encode4(y + 16 * h + 12));
  return Fp8Meta{scale, expand, smm};
}

}  // namespace mmuon
