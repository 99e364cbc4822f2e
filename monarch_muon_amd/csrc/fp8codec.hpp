// FP8 (OCP e4m3fn or e5m2, group-128, dynamic range expansion) optimizer-state
// codec.
//
// Device restatement of the codec of coat_state_muon.py:22-91 (itself the
// first/second-order half of COAT's AdamW expand kernel), for both formats the
// reference maps (coat_state_muon.py:17) and any expand_min (:113, :123).  Each
// group of 128 consecutive elements carries fp32 scale, expand and
// sqrt_minmax.  A group is held by a few lanes of a wave, a run of consecutive
// elements per lane.
//
// Per element the work is written for the VALU budget of an HBM-streaming
// kernel: the dequantizer's power |raw s|^(1/expand) is one exp2 of
// (log2|raw| + log2 s) / expand (log2 s / expand once per group), and the
// quantizer's (|x| / smm)^expand / scale one exp2 of
// expand log2(|x| / smm) - log2 scale.  Each fast path is taken only where the
// reference's clamps to 1e-30 cannot act (checked once per group); the other
// groups, and partial groups, run an exact restatement with the clamps.
#pragma once

#include "common.hpp"

namespace mmuon {

constexpr float QEPS = 1e-30f;
constexpr float LOG2_QEPS = -99.657842847f;  // log2(QEPS)

// ---------------------------------------------------------------------------
// Formats.  gfx950's v_cvt_f32_fp8 / v_cvt_pk_fp8_f32 (e4m3fn) and
// v_cvt_f32_bf8 / v_cvt_pk_bf8_f32 (e5m2) convert the OCP formats with
// round-to-nearest-even (the rounding torch's float8 casts use); the encoder's
// inputs are clamped to +-MAX first, as the codec saturates.
// ---------------------------------------------------------------------------
struct E4M3 {
  static constexpr int CODE = MMUON_F8E4M3;
  static constexpr float MAX = 448.0f;        // torch.finfo(float8_e4m3fn).max
  static constexpr float MIN_SUB = 0x1p-9f;   // smallest non-zero magnitude
  template <int B>
  static __device__ __forceinline__ float cvt(uint32_t c) { return __builtin_amdgcn_cvt_f32_fp8(int(c), B); }
  static __device__ __forceinline__ int cvt_pk(float a, float b, int old, bool hi) {
    return hi ? __builtin_amdgcn_cvt_pk_fp8_f32(a, b, old, true) : __builtin_amdgcn_cvt_pk_fp8_f32(a, b, old, false);
  }
};
struct E5M2 {
  static constexpr int CODE = MMUON_F8E5M2;
  static constexpr float MAX = 57344.0f;      // torch.finfo(float8_e5m2).max
  static constexpr float MIN_SUB = 0x1p-16f;
  template <int B>
  static __device__ __forceinline__ float cvt(uint32_t c) { return __builtin_amdgcn_cvt_f32_bf8(int(c), B); }
  static __device__ __forceinline__ int cvt_pk(float a, float b, int old, bool hi) {
    return hi ? __builtin_amdgcn_cvt_pk_bf8_f32(a, b, old, true) : __builtin_amdgcn_cvt_pk_bf8_f32(a, b, old, false);
  }
};

// one code byte (in the low byte of c) -> fp32 (exact)
template <class F>
__device__ __forceinline__ float fp8_decode(uint32_t c) { return F::template cvt<0>(c); }

template <class F>
__device__ __forceinline__ void decode4(uint32_t c, float* v) {
  v[0] = F::template cvt<0>(c);
  v[1] = F::template cvt<1>(c);
  v[2] = F::template cvt<2>(c);
  v[3] = F::template cvt<3>(c);
}
// values already clamped to [-MAX, MAX]
template <class F>
__device__ __forceinline__ uint32_t encode4(const float* v) {
  int w = F::cvt_pk(v[0], v[1], 0, false);
  w = F::cvt_pk(v[2], v[3], w, true);
  return uint32_t(w);
}

struct Fp8Meta {
  float scale, expand, sqrt_minmax;
};

// x^y for a positive normal x, as 2^(y log2 x) with the hardware base-2
// logarithm and exponential (v_log_f32, v_exp_f32).  Rounding the product
// y log2 x adds a relative error of about |y log2 x| * 2^-24 to the result.
__device__ __forceinline__ float pow_pos(float x, float y) {
  return __builtin_amdgcn_exp2f(y * __builtin_amdgcn_logf(x));
}

// ---------------------------------------------------------------------------
// Dequantization (coat_state_muon.py:22-43).  Per group: ie = 1/max(expand,
// QEPS), smm = max(sqrt_minmax, QEPS).  A non-zero code decodes to
// |raw| >= MIN_SUB, so where scale >= QEPS / MIN_SUB the clamp
// max(|raw scale|, QEPS) never acts, and the value is
//   sign(raw) 2^(ie log2|raw| + ie log2 scale) smm
// with log2|raw| = -inf (value 0) for a zero code.  Other groups (scale
// below that, or not finite) run the restatement with the clamp.
// ---------------------------------------------------------------------------
struct Fp8Dq {
  float ie;     // 1 / max(expand, QEPS)
  float c;      // ie log2(scale)   (fast groups)
  float scale;
  float smm;    // max(sqrt_minmax, QEPS)
  bool fast;
};
template <class F>
__device__ __forceinline__ Fp8Dq fp8_dq(const Fp8Meta& md) {
  Fp8Dq d;
  d.ie = 1.0f / fmaxf(md.expand, QEPS);
  d.scale = md.scale;
  d.smm = fmaxf(md.sqrt_minmax, QEPS);
  d.fast = md.scale >= QEPS / F::MIN_SUB && md.scale <= 3.4028235e38f;
  d.c = d.ie * __builtin_amdgcn_logf(d.fast ? md.scale : 1.0f);
  return d;
}

// one element, the exact restatement (every group)
__device__ __forceinline__ float fp8_dequant_exact(float raw, const Fp8Dq& d, bool sgn) {
  if (sgn) {
    const float scaled = raw * d.scale;
    const float absolute = fabsf(scaled);
    const float s = scaled >= 0.f ? 1.f : -1.f;
    const float power = pow_pos(fmaxf(absolute, QEPS), d.ie);
    return absolute > 0.f ? (s * power) * d.smm : 0.f;
  }
  const float scaled = fmaxf(raw * d.scale, 0.f);
  const float power = pow_pos(fmaxf(scaled, QEPS), d.ie);
  return scaled > 0.f ? power * d.smm : 0.f;
}

// one element of a fast group (a code of +-0 decodes to +0, as in the
// reference)
__device__ __forceinline__ float fp8_dequant_fast(float raw, const Fp8Dq& d, bool sgn) {
  if (sgn) {
    const float v = __builtin_amdgcn_exp2f(fmaf(d.ie, __builtin_amdgcn_logf(fabsf(raw)), d.c)) * d.smm;
    return raw < 0.f ? -v : v;
  }
  const float p = __builtin_amdgcn_exp2f(fmaf(d.ie, __builtin_amdgcn_logf(fmaxf(raw, 0.f)), d.c));
  return p * d.smm;
}

template <class F>
__device__ __forceinline__ float fp8_dequant(uint32_t code, const Fp8Meta& md, bool sgn) {
  const Fp8Dq d = fp8_dq<F>(md);
  const float raw = fp8_decode<F>(code);
  return d.fast ? fp8_dequant_fast(raw, d, sgn) : fp8_dequant_exact(raw, d, sgn);
}

// This lane's E elements of one group (E a multiple of 16: whole 16-byte code
// accesses).  Codes of elements that do not exist must be zero (they decode to
// zero).
template <class F, int E>
__device__ __forceinline__ void fp8_dequant_lane(const uint4 (&codes)[E / 16], const Fp8Dq& d, bool sgn,
                                                 float (&out)[E]) {
  float raw[E];
#pragma unroll
  for (int h = 0; h < E / 16; ++h) {
    decode4<F>(codes[h].x, raw + 16 * h);
    decode4<F>(codes[h].y, raw + 16 * h + 4);
    decode4<F>(codes[h].z, raw + 16 * h + 8);
    decode4<F>(codes[h].w, raw + 16 * h + 12);
  }
  if (d.fast) {
#pragma unroll
    for (int k = 0; k < E; ++k) out[k] = fp8_dequant_fast(raw[k], d, sgn);
  } else {
#pragma unroll
    for (int k = 0; k < E; ++k) out[k] = fp8_dequant_exact(raw[k], d, sgn);
  }
}

// ---------------------------------------------------------------------------
// Cross-lane max / min over the 128/E lanes of a group (every lane of the
// group active): swap neighbours, swap pairs (, mirror the halves of 8).
// ---------------------------------------------------------------------------
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
  return __builtin_amdgcn_mov_dpp(v, CTRL, 0xf, 0xf, false);
}
template <int LANES>
__device__ __forceinline__ float group_max(float v) {
  static_assert(LANES == 4 || LANES == 8, "groups of 4 or 8 lanes");
  v = fmaxf(v, __int_as_float(dpp_i<0xb1>(__float_as_int(v))));                      // quad_perm [1,0,3,2]
  v = fmaxf(v, __int_as_float(dpp_i<0x4e>(__float_as_int(v))));                      // quad_perm [2,3,0,1]
  if constexpr (LANES == 8) v = fmaxf(v, __int_as_float(dpp_i<0x141>(__float_as_int(v))));  // row_half_mirror
  return v;
}
template <int LANES>
__device__ __forceinline__ uint32_t group_min_u32(uint32_t v) {
  static_assert(LANES == 4 || LANES == 8, "groups of 4 or 8 lanes");
  v = min(v, uint32_t(dpp_i<0xb1>(int(v))));
  v = min(v, uint32_t(dpp_i<0x4e>(int(v))));
  if constexpr (LANES == 8) v = min(v, uint32_t(dpp_i<0x141>(int(v))));
  return v;
}

// ---------------------------------------------------------------------------
// Quantization (coat_state_muon.py:46-91) of one group: this lane's E values
// (nvalid of them exist: FULL means all E, in every lane of the group).
// Returns the group metadata (valid in every lane of the group) and this
// lane's E codes.  emin: expand_min.
//
// The group's smallest non-zero |x| is found as the smallest unsigned
// (bits(x) << 1) - 1, which is monotone in |x| and maps +-0 to the largest
// value.  Per element, in a group where amin / smm >= QEPS (so the clamp
// max(|x| / smm, QEPS) acts on no non-zero element) and expand <= 32:
//   q = sign(x) 2^(expand log2(|x| (1/smm)) - log2 scale)
// (a zero, +0 or -0, gives 2^-inf = +0, the reference's 0; a negative value
// that rounds to zero keeps its sign, -0, as in the reference); a group with a larger expand (values within a
// factor ~1.4 of each other, where expand magnifies the rounding of |x|/smm)
// divides |x| / smm exactly first.  Other groups run the restatement with the
// clamp.
// ---------------------------------------------------------------------------
template <class F, int E, bool FULL>
__device__ __forceinline__ Fp8Meta fp8_quant_group(const float (&x)[E], int nvalid, bool sgn, float emin,
                                                   uint4 (&codes)[E / 16]) {
  float amax = 0.f;
  uint32_t kmin = 0xffffffffu;
#pragma unroll
  for (int k = 0; k < E; ++k) {
    if (FULL || k < nvalid) {
      amax = fmaxf(amax, fabsf(x[k]));
      kmin = min(kmin, (__float_as_uint(x[k]) << 1) - 1u);
    }
  }
  amax = fmaxf(group_max<128 / E>(amax), QEPS);
  float amin = __uint_as_float((group_min_u32<128 / E>(kmin) + 1u) >> 1);   // 0: no non-zero value
  amin = amin > 0.f ? fmaxf(amin, QEPS) : QEPS;
  float ratio = amax / amin;
  ratio = fmaxf(ratio, 1.0f + QEPS);
  const float ratio_upper = F::MAX * F::MAX / 2.0f;
  const float log_ratio = log2f(ratio);
  const float safe_log = log_ratio > QEPS ? log_ratio : 1.0f;
  const float raw_expand = floorf((log2f(ratio_upper) / safe_log) * emin) / emin;
  const float expand = ratio <= 1.0f + QEPS ? 1.0f : fmaxf(raw_expand, 1.0f / emin);
  const float smm = fmaxf(sqrtf(amax) * sqrtf(amin), QEPS);
  const float scale = fmaxf(pow_pos(fmaxf(amax / smm, QEPS), expand) / F::MAX, QEPS);
  const float inv_smm = 1.0f / smm;
  const float lsc = __builtin_amdgcn_logf(scale);
  float y[E];
  if (FULL && amin * inv_smm >= QEPS) {
    if (expand <= 32.0f) {
#pragma unroll
      for (int k = 0; k < E; ++k) {
        const float np = __builtin_amdgcn_exp2f(fmaf(expand, __builtin_amdgcn_logf(fabsf(x[k]) * inv_smm), -lsc));
        y[k] = __builtin_amdgcn_fmed3f(sgn && x[k] < 0.f ? -np : np, -F::MAX, F::MAX);
      }
    } else {
#pragma unroll
      for (int k = 0; k < E; ++k) {
        const float np = __builtin_amdgcn_exp2f(fmaf(expand, __builtin_amdgcn_logf(fabsf(x[k]) / smm), -lsc));
        y[k] = __builtin_amdgcn_fmed3f(sgn && x[k] < 0.f ? -np : np, -F::MAX, F::MAX);
      }
    }
  } else {
#pragma unroll
    for (int k = 0; k < E; ++k) {
      const float a = fabsf(x[k]);
      const float np = pow_pos(fmaxf(a / smm, QEPS), expand) / scale;
      float nrm = 0.f;
      if ((FULL || k < nvalid) && a > 0.f) nrm = sgn ? copysignf(np, x[k]) : np;
      y[k] = __builtin_amdgcn_fmed3f(nrm, -F::MAX, F::MAX);
    }
  }
#pragma unroll
  for (int h = 0; h < E / 16; ++h)
    codes[h] = make_uint4(encode4<F>(y + 16 * h), encode4<F>(y + 16 * h + 4), encode4<F>(y + 16 * h + 8),
                          encode4<F>(y + 16 * h + 12));
  return Fp8Meta{scale, expand, smm};
}

}  // namespace mmuon
