// FP8 (OCP e4m3fn, group-128, dynamic range expansion) optimizer-state codec.
//
// Device restatement of the codec of coat_state_muon.py:22-91 (itself the
// first/second-order half of COAT's AdamW expand kernel).  Each group of 128
// consecutive elements carries fp32 scale, expand and sqrt_minmax.  One wave64
// owns one group, two elements per lane (lane and lane+64).
#pragma once

#include "common.hpp"

namespace mmuon {

constexpr float FP8_MAX = 448.0f;
constexpr float QEPS = 1e-30f;
constexpr float EXPAND_MIN = 16.0f;

// fp32 -> e4m3fn byte: round to nearest even, saturating at +-448, NaN -> 0x7f.
__device__ __forceinline__ uint8_t e4m3_encode(float x) {
  const uint32_t u = __float_as_uint(x);
  const uint32_t sign = (u >> 24) & 0x80u;
  float a = fabsf(x);
  if (a != a) return uint8_t(0x7fu | sign);
  a = fminf(a, FP8_MAX);
  if (a < 0.015625f) {                       // below 2^-6: multiples of 2^-9
    const float k = rintf(a * 512.0f);       // exact scaling, RNE; k == 8 is the min normal
    return uint8_t(sign | uint32_t(k));
  }
  const uint32_t au = __float_as_uint(a);
  uint32_t e = (au >> 23) - 127u + 7u;
  const uint32_t man = au & 0x7fffffu;
  uint32_t q = man >> 20;
  const uint32_t rem = man & 0xfffffu;
  q += (rem > 0x80000u) || (rem == 0x80000u && (q & 1u));
  if (q == 8u) {
    q = 0u;
    e += 1u;
  }
  return uint8_t(sign | (e << 3) | q);
}

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

// coat_state_muon.py:22-43 for one element.
__device__ __forceinline__ float fp8_dequant(uint32_t code, const Fp8Meta& md, bool sgn) {
  const float ex = fmaxf(md.expand, QEPS);
  const float smm = fmaxf(md.sqrt_minmax, QEPS);
  const float inv = 1.0f / ex;
  const float raw = e4m3_decode(code);
  if (sgn) {
    const float scaled = raw * md.scale;
    const float absolute = fabsf(scaled);
    const float s = scaled >= 0.f ? 1.f : -1.f;
    const float power = powf(fmaxf(absolute, QEPS), inv);
    return absolute > 0.f ? (s * power) * smm : 0.f;
  }
  const float scaled = fmaxf(raw * md.scale, 0.f);
  const float power = powf(fmaxf(scaled, QEPS), inv);
  return scaled > 0.f ? power * smm : 0.f;
}

// coat_state_muon.py:46-91 for one group held by a whole wave (two elements
// per lane; v0/v1 say whether the element exists).  Returns the codes of this
// lane's two elements and the group metadata (valid in every lane).
__device__ __forceinline__ Fp8Meta fp8_quant_group(float x0, float x1, bool v0, bool v1, bool sgn,
                                                   uint8_t& q0, uint8_t& q1) {
  const float a0 = fabsf(x0), a1 = fabsf(x1);
  float amax = fmaxf(v0 ? a0 : 0.f, v1 ? a1 : 0.f);
  const bool n0 = v0 && a0 > 0.f, n1 = v1 && a1 > 0.f;
  float amin = fminf(n0 ? a0 : 3.4028235e38f, n1 ? a1 : 3.4028235e38f);
  const int nz = wave_isum(int(n0) + int(n1));
  amax = wave_max(amax);
  amin = wave_min(amin);
  amax = fmaxf(amax, QEPS);
  amin = nz > 0 ? fmaxf(amin, QEPS) : QEPS;
  float ratio = amax / amin;
  ratio = fmaxf(ratio, 1.0f + QEPS);
  const float ratio_upper = FP8_MAX * FP8_MAX / 2.0f;
  const float log_ratio = log2f(ratio);
  const float safe_log = log_ratio > QEPS ? log_ratio : 1.0f;
  const float raw_expand = floorf((log2f(ratio_upper) / safe_log) * EXPAND_MIN) / EXPAND_MIN;
  const float expand = ratio <= 1.0f + QEPS ? 1.0f : fmaxf(raw_expand, 1.0f / EXPAND_MIN);
  const float smm = fmaxf(sqrtf(amax) * sqrtf(amin), QEPS);
  const float scale = fmaxf(powf(fmaxf(amax / smm, QEPS), expand) / FP8_MAX, QEPS);
  auto enc = [&](float x, float a, bool valid) -> uint8_t {
    const float np = powf(fmaxf(a / smm, QEPS), expand);
    float nrm = 0.f;
    if (valid && a > 0.f) nrm = sgn ? (x >= 0.f ? np : -np) : np;
    return e4m3_encode(nrm / scale);
  };
  q0 = enc(x0, a0, v0);
  q1 = enc(x1, a1, v1);
  return Fp8Meta{scale, expand, smm};
}

}  // namespace mmuon
