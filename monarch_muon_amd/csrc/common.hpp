// Shared device helpers for the gfx950 Monarch-Muon kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/mmuon.h"
#include "addr.hpp"

namespace mmuon {

// p made wave-uniform: both address words read from the first active lane
// and joined as unsigned words (join_words).
template <class T>
__device__ __forceinline__ T* uniform_ptr(T* p) {
  const uint64_t a = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = uint32_t(__builtin_amdgcn_readfirstlane(int(low_word(a))));
  const uint32_t hi = uint32_t(__builtin_amdgcn_readfirstlane(int(high_word(a))));
  return reinterpret_cast<T*>(join_words(lo, hi));
}

// ---------------------------------------------------------------------------
// bf16 <-> fp32.  bf16 is carried as its raw 16-bit pattern; conversion is
// round-to-nearest-even (the rounding torch uses for every bf16 tensor op).
// ---------------------------------------------------------------------------
__device__ __forceinline__ float bf2f(uint16_t h) { return __uint_as_float(uint32_t(h) << 16); }

// gfx950 converts with v_cvt_pk_bf16_f32 (round to nearest even).
__device__ __forceinline__ uint16_t f2bf(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}

// two floats -> packed bf16 pair (lo = a), one v_cvt_pk_bf16_f32
__device__ __forceinline__ uint32_t f2bf2(float a, float b) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  const bf16x2_t v = {static_cast<__bf16>(a), static_cast<__bf16>(b)};
  return __builtin_bit_cast(uint32_t, v);
}

// round a float to bf16 precision and back
__device__ __forceinline__ float rbf(float f) { return bf2f(f2bf(f)); }

// ---------------------------------------------------------------------------
// Newton-Schulz workspace layout.  bf16 stacks (X, Gram, polynomial) are kept
// in 32-column panels: element (i, j) of a matrix with R rows sits at
//   (j / 32) * (R * 32) + i * 32 + j % 32,
// so the 32-wide K slice of 256 rows that an MFMA stage loads is one contiguous
// 16 KiB run.  fp32 stacks are plain row-major [R][cols].
// ---------------------------------------------------------------------------
constexpr int PANEL = 32;

__host__ __device__ __forceinline__ int64_t panel_off(int64_t rows, int64_t i, int64_t j) {
  return (j >> 5) * (rows << 5) + (i << 5) + (j & 31);
}

// Element access by storage type tag.
// xoff(mp, np, i, j): offset of X-stack element (i, j) within one block.
struct F32T {
  using storage = float;
  static __device__ __forceinline__ float load(const float* p, int64_t i) { return p[i]; }
  static __device__ __forceinline__ void store(float* p, int64_t i, float v) { p[i] = v; }
  static __device__ __forceinline__ float round(float v) { return v; }
  static __device__ __forceinline__ int64_t xoff(int mp, int np, int64_t i, int64_t j) {
    (void)mp;
    return i * np + j;
  }
};
struct BF16T {
  using storage = uint16_t;
  static __device__ __forceinline__ float load(const uint16_t* p, int64_t i) { return bf2f(p[i]); }
  static __device__ __forceinline__ void store(uint16_t* p, int64_t i, float v) { p[i] = f2bf(v); }
  static __device__ __forceinline__ float round(float v) { return rbf(v); }
  static __device__ __forceinline__ int64_t xoff(int mp, int np, int64_t i, int64_t j) {
    (void)np;
    return panel_off(mp, i, j);
  }
};

// 16-B non-temporal (streaming) access: data read or written once per pass
typedef unsigned int u32x4_nt __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 load16_nt(const void* p) {
  const u32x4_nt r = __builtin_nontemporal_load(reinterpret_cast<const u32x4_nt*>(p));
  return make_uint4(r.x, r.y, r.z, r.w);
}
__device__ __forceinline__ void store16_nt(void* p, const uint4& v) {
  const u32x4_nt r = {v.x, v.y, v.z, v.w};
  __builtin_nontemporal_store(r, reinterpret_cast<u32x4_nt*>(p));
}

// 8 consecutive elements, vector access (16-B aligned); *_nt: non-temporal
template <class T>
struct Vec8;
template <>
struct Vec8<BF16T> {
  static __device__ __forceinline__ void unpack(const uint4& r, float v[8]) {
    const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      v[2 * q] = __uint_as_float(w[q] << 16);
      v[2 * q + 1] = __uint_as_float(w[q] & 0xffff0000u);
    }
  }
  static __device__ __forceinline__ uint4 pack(const float v[8]) {
    uint4 r;
    r.x = uint32_t(f2bf(v[0])) | (uint32_t(f2bf(v[1])) << 16);
    r.y = uint32_t(f2bf(v[2])) | (uint32_t(f2bf(v[3])) << 16);
    r.z = uint32_t(f2bf(v[4])) | (uint32_t(f2bf(v[5])) << 16);
    r.w = uint32_t(f2bf(v[6])) | (uint32_t(f2bf(v[7])) << 16);
    return r;
  }
  static __device__ __forceinline__ void load(const uint16_t* p, float v[8]) {
    unpack(*reinterpret_cast<const uint4*>(p), v);
  }
  static __device__ __forceinline__ void store(uint16_t* p, const float v[8]) {
    *reinterpret_cast<uint4*>(p) = pack(v);
  }
  static __device__ __forceinline__ void load_nt(const uint16_t* p, float v[8]) { unpack(load16_nt(p), v); }
  static __device__ __forceinline__ void store_nt(uint16_t* p, const float v[8]) { store16_nt(p, pack(v)); }
};
template <>
struct Vec8<F32T> {
  static __device__ __forceinline__ void load(const float* p, float v[8]) {
    const float4 a = reinterpret_cast<const float4*>(p)[0];
    const float4 b = reinterpret_cast<const float4*>(p)[1];
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  }
  static __device__ __forceinline__ void store(float* p, const float v[8]) {
    reinterpret_cast<float4*>(p)[0] = make_float4(v[0], v[1], v[2], v[3]);
    reinterpret_cast<float4*>(p)[1] = make_float4(v[4], v[5], v[6], v[7]);
  }
  static __device__ __forceinline__ void load_nt(const float* p, float v[8]) {
    const uint4 a = load16_nt(p), b = load16_nt(p + 4);
    v[0] = __uint_as_float(a.x); v[1] = __uint_as_float(a.y); v[2] = __uint_as_float(a.z); v[3] = __uint_as_float(a.w);
    v[4] = __uint_as_float(b.x); v[5] = __uint_as_float(b.y); v[6] = __uint_as_float(b.z); v[7] = __uint_as_float(b.w);
  }
  static __device__ __forceinline__ void store_nt(float* p, const float v[8]) {
    store16_nt(p, make_uint4(__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]), __float_as_uint(v[3])));
    store16_nt(p + 4, make_uint4(__float_as_uint(v[4]), __float_as_uint(v[5]), __float_as_uint(v[6]), __float_as_uint(v[7])));
  }
};

// ---------------------------------------------------------------------------
// wave64 reductions (cross-lane through ds_swizzle/DPP as the compiler picks)
// ---------------------------------------------------------------------------
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ __forceinline__ float wave_min(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fminf(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ __forceinline__ int wave_isum(int v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Block-wide sum for blockDim.x == NT (multiple of 64); result valid in thread 0.
template <int NT>
__device__ __forceinline__ float block_sum(float v, float* scratch /* NT/64 floats */) {
  v = wave_sum(v);
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  if (lane == 0) scratch[wid] = v;
  __syncthreads();
  float r = 0.f;
  if (threadIdx.x == 0) {
#pragma unroll
    for (int w = 0; w < NT / 64; ++w) r += scratch[w];
  }
  return r;
}

}  // namespace mmuon
