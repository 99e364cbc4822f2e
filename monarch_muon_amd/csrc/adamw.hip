// Embedded AdamW of the Monarch-Muon optimizer as one multi-tensor launch.
//
// Per element, in the reference's op order (membench monarch_muon.py:196-208):
//   p  <- R_p(p * (1 - lr wd))                         (when wd > 0)
//   m  <- R_s(m * b1) ; m <- R_s(m + (1-b1) g)         (foreach add with alpha: fused)
//   v  <- R_s(v * b2) ; v <- R_s(v + (1-b2) (g g))     (addcmul)
//   d  <- R_s(sqrt v) ; d <- R_s(d / sqrt(bc2)) ; d <- R_s(d + eps)
//   p  <- R_p(p + (-lr/bc1) (m / d))                   (addcdiv)
// R_x rounds to the tensor's dtype.  Algorithmic HBM traffic, bf16 p/g/m/v:
// 14 B per element.
#include "common.hpp"
#include "fp8codec.hpp"
#include "kernels.hpp"

namespace mmuon {

// The roundings are where torch's ops round; within an op, the fp32 formula
// torch's GPU kernels evaluate, found bit for bit against its foreach and
// per-tensor ops on the GPU: add with alpha is fma(g, alpha, m), addcmul
// fma(value, g g, v), addcdiv fma(value, m / d, p).  The division by
// sqrt(bc2) is a true division (torch's foreach div; its per-tensor div by a
// scalar multiplies by the fp32 reciprocal, which for beta2 = 0.95 gives the
// same bf16 result at every bf16 value and step count up to 20000).
template <class TP, class TS>
__device__ __forceinline__ void adamw_elem(float& p, float g, float& m, float& v, const AdamWArgs& a) {
  if (a.apply_wd) p = TP::round(p * a.wd_factor);
  m = TS::round(m * a.beta1);
  m = TS::round(fmaf(g, a.one_minus_beta1, m));
  v = TS::round(v * a.beta2);
  v = TS::round(fmaf(a.one_minus_beta2, g * g, v));
  float d = TS::round(sqrtf(v));
  d = TS::round(d / a.sqrt_bc2);
  d = TS::round(d + a.eps);
  p = TP::round(fmaf(a.neg_step_size, m / d, p));
}

// The same update for the FP8-state kernel, whose moments are fp32 values of a
// format held to a tolerance, not bit for bit: the square root and the two
// quotients use the hardware's 1-ulp v_sqrt_f32 and v_rcp_f32 (with a multiply
// by the host's fp32 1/sqrt(bc2)) in place of the correctly rounded sequences
// (the kernel issues 77 VALU instructions per element with them, 114 without).
// Only the parameter update depends on them; the moments and their codes do
// not.  Used
// where eps sqrt(bc2) >= 2^-37 (AdamWArgs::fast_quot): then d >= eps is normal,
// and the root of a subnormal v (below 2^-63, which v_sqrt_f32 may flush to
// zero), divided by sqrt(bc2), is below half an ulp of eps, so d + eps rounds
// to eps either way.
template <class TP, class TS>
__device__ __forceinline__ void adamw_elem_fast(float& p, float g, float& m, float& v, const AdamWArgs& a) {
  if (a.apply_wd) p = TP::round(p * a.wd_factor);
  m = TS::round(m * a.beta1);
  m = TS::round(fmaf(g, a.one_minus_beta1, m));
  v = TS::round(v * a.beta2);
  v = TS::round(fmaf(a.one_minus_beta2, g * g, v));
  float d = TS::round(__builtin_amdgcn_sqrtf(v));
  d = TS::round(d * a.inv_sqrt_bc2);
  d = TS::round(d + a.eps);
  p = TP::round(fmaf(a.neg_step_size, m * __builtin_amdgcn_rcpf(d), p));
}

constexpr int ADAM_NT = 256;

template <class TP, class TG, class TS>
__global__ __launch_bounds__(ADAM_NT) void adamw_kernel(AdamWArgs a) {
  const int64_t code = a.chunks[blockIdx.x];
  const int t = int(code >> 40);
  const int64_t start = code & ((int64_t(1) << 40) - 1);
  const mmuon_adamw_tensor T = a.tensors[t];
  const int64_t end = min(T.numel, start + int64_t(a.chunk_elems));
  auto* p = reinterpret_cast<typename TP::storage*>(T.param);
  const auto* g = reinterpret_cast<const typename TG::storage*>(T.grad);
  auto* m = reinterpret_cast<typename TS::storage*>(T.exp_avg);
  auto* v = reinterpret_cast<typename TS::storage*>(T.exp_avg_sq);
  const GradClip clip = grad_clip(a.gscale);
  int64_t tail = start;
  // 8 elements per thread and 16-B accesses when all four streams are aligned
  // here; two groups' loads are issued before either is computed; every access
  // is non-temporal (each element is read and written once per step)
  const uintptr_t al = reinterpret_cast<uintptr_t>(p + start) | reinterpret_cast<uintptr_t>(g + start) |
                       reinterpret_cast<uintptr_t>(m + start) | reinterpret_cast<uintptr_t>(v + start);
  if ((al & 15) == 0) {
    const int64_t stop = start + ((end - start) & ~int64_t(7));
    for (int64_t i0 = start + int64_t(threadIdx.x) * 8; i0 < stop; i0 += 2 * ADAM_NT * 8) {
      const int64_t i1 = i0 + ADAM_NT * 8;
      const bool two = i1 < stop;
      float P[2][8], G[2][8], M[2][8], V[2][8];
      Vec8<TP>::load_nt(p + i0, P[0]);
      Vec8<TG>::load_nt(g + i0, G[0]);
      Vec8<TS>::load_nt(m + i0, M[0]);
      Vec8<TS>::load_nt(v + i0, V[0]);
      if (two) {
        Vec8<TP>::load_nt(p + i1, P[1]);
        Vec8<TG>::load_nt(g + i1, G[1]);
        Vec8<TS>::load_nt(m + i1, M[1]);
        Vec8<TS>::load_nt(v + i1, V[1]);
      }
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        if (h == 1 && !two) break;
        const int64_t i = h ? i1 : i0;
        clip_grads<TG>(G[h], clip);
#pragma unroll
        for (int e = 0; e < 8; ++e) adamw_elem<TP, TS>(P[h][e], G[h][e], M[h][e], V[h][e], a);
        Vec8<TP>::store_nt(p + i, P[h]);
        Vec8<TS>::store_nt(m + i, M[h]);
        Vec8<TS>::store_nt(v + i, V[h]);
      }
    }
    tail = stop;
  }
  for (int64_t i = tail + threadIdx.x; i < end; i += ADAM_NT) {
    float pv = TP::load(p, i), mv = TS::load(m, i), vv = TS::load(v, i);
    adamw_elem<TP, TS>(pv, clipped<TG>(TG::load(g, i), clip), mv, vv, a);
    TP::store(p, i, pv);
    TS::store(m, i, mv);
    TS::store(v, i, vv);
  }
}

int launch_adamw(const AdamWArgs& a, int param_dtype, int grad_dtype, int state_dtype,
                 hipStream_t s) {
  if (a.nchunks <= 0) return 0;
  const dim3 grid(unsigned(a.nchunks)), block(ADAM_NT);
#define MMUON_ADAM_CASE(PD, GD, SD, TP, TG, TS)                                  \
  if (param_dtype == PD && grad_dtype == GD && state_dtype == SD) {              \
    hipLaunchKernelGGL((adamw_kernel<TP, TG, TS>), grid, block, 0, s, a);        \
    return 0;                                                                    \
  }
  MMUON_ADAM_CASE(MMUON_BF16, MMUON_BF16, MMUON_BF16, BF16T, BF16T, BF16T)
  MMUON_ADAM_CASE(MMUON_BF16, MMUON_BF16, MMUON_F32, BF16T, BF16T, F32T)
  MMUON_ADAM_CASE(MMUON_F32, MMUON_F32, MMUON_F32, F32T, F32T, F32T)
  MMUON_ADAM_CASE(MMUON_F32, MMUON_F32, MMUON_BF16, F32T, F32T, BF16T)
#undef MMUON_ADAM_CASE
  return -1;
}

// ---------------------------------------------------------------------------
// FP8-state AdamW: one 128-element metadata group per F8_LANES (8) lanes,
// F8_ELEMS (16) consecutive elements per lane (32 per lane, which shares each
// group's metadata work among more elements, takes 190 VGPRs, two waves per
// SIMD, and measured 5% slower); the moments are dequantized to fp32,
// updated in fp32 (the reference's dequantized states are fp32 tensors), and
// requantized (exp_avg signed in format FM, exp_avg_sq unsigned in format FV:
// the reference's first_order_bit / second_order_bit, coat_state_muon.py:121-122).
// Moments created in this step (have_state 0) start at zero in the parameter
// dtype and every moment op rounds to it (TS = TP), as the wrapped step's
// zeros_like(param) states do (coat_state_muon.py:126-139 around membench
// monarch_muon.py:184-190).  chunk = tensor << 40 | first element of the group;
// a tensor's last group may be short (numel % 128 != 0).
// ---------------------------------------------------------------------------
constexpr int F8_ELEMS = 16, F8_LANES = 128 / F8_ELEMS;
constexpr int F8_GPW = ADAM_NT / F8_LANES;  // groups per workgroup

template <class T>
__device__ __forceinline__ void load_lane(const typename T::storage* p, int64_t e0, int nvalid, bool vec,
                                          float v[F8_ELEMS]) {
  if (vec) {
#pragma unroll
    for (int h = 0; h < F8_ELEMS / 8; ++h) Vec8<T>::load(p + e0 + 8 * h, v + 8 * h);
    return;
  }
#pragma unroll
  for (int k = 0; k < F8_ELEMS; ++k) v[k] = k < nvalid ? T::load(p, e0 + k) : 0.f;
}
__device__ __forceinline__ void load_codes(const uint8_t* q, int64_t e0, int nvalid, bool vec,
                                           uint4 (&c)[F8_ELEMS / 16]) {
  if (vec) {
#pragma unroll
    for (int h = 0; h < F8_ELEMS / 16; ++h) c[h] = *reinterpret_cast<const uint4*>(q + e0 + 16 * h);
    return;
  }
  uint32_t w[F8_ELEMS / 4] = {};
#pragma unroll
  for (int k = 0; k < F8_ELEMS; ++k)
    if (k < nvalid) w[k >> 2] |= uint32_t(q[e0 + k]) << (8 * (k & 3));
#pragma unroll
  for (int h = 0; h < F8_ELEMS / 16; ++h) c[h] = make_uint4(w[4 * h], w[4 * h + 1], w[4 * h + 2], w[4 * h + 3]);
}
__device__ __forceinline__ void store_codes(uint8_t* q, int64_t e0, int nvalid, bool vec,
                                            const uint4 (&c)[F8_ELEMS / 16]) {
  if (vec) {
#pragma unroll
    for (int h = 0; h < F8_ELEMS / 16; ++h) *reinterpret_cast<uint4*>(q + e0 + 16 * h) = c[h];
    return;
  }
#pragma unroll
  for (int k = 0; k < F8_ELEMS; ++k) {
    const uint4& u = c[k >> 4];
    const uint32_t w = (k & 15) < 4 ? u.x : (k & 15) < 8 ? u.y : (k & 15) < 12 ? u.z : u.w;
    if (k < nvalid) q[e0 + k] = uint8_t(w >> (8 * (k & 3)));
  }
}

template <class TP, class TG, class TS, class FM, class FV, bool FASTQ>
__global__ __launch_bounds__(ADAM_NT) void adamw_fp8_kernel(AdamWArgs a) {
  const int64_t gidx = int64_t(blockIdx.x) * F8_GPW + (threadIdx.x / F8_LANES);
  if (gidx >= a.nchunks) return;  // a group's lanes leave together
  const int sub = threadIdx.x % F8_LANES;
  const int64_t code = a.chunks[gidx];
  const int t = int(code >> 40);
  const int64_t start = code & ((int64_t(1) << 40) - 1);
  const mmuon_adamw_tensor T = a.tensors[t];
  const mmuon_adamw_fp8_tensor M = a.fp8[t];
  const int64_t grp = start >> 7;
  auto* p = reinterpret_cast<typename TP::storage*>(T.param);
  const auto* g = reinterpret_cast<const typename TG::storage*>(T.grad);
  uint8_t* qm = reinterpret_cast<uint8_t*>(T.exp_avg);
  uint8_t* qv = reinterpret_cast<uint8_t*>(T.exp_avg_sq);
  const int64_t e0 = start + sub * F8_ELEMS;
  const int nvalid = int(max(int64_t(0), min(int64_t(F8_ELEMS), T.numel - e0)));
  const bool full = start + 128 <= T.numel;  // uniform over the group's lanes
  // 16-B parameter / gradient / code accesses for a full, aligned lane
  const uintptr_t al = reinterpret_cast<uintptr_t>(p + e0) | reinterpret_cast<uintptr_t>(g + e0) |
                       reinterpret_cast<uintptr_t>(qm + e0) | reinterpret_cast<uintptr_t>(qv + e0);
  const bool vec = nvalid == F8_ELEMS && (al & 15) == 0;
  float pv[F8_ELEMS], gv[F8_ELEMS], m[F8_ELEMS], v[F8_ELEMS];
  load_lane<TP>(p, e0, nvalid, vec, pv);
  load_lane<TG>(g, e0, nvalid, vec, gv);
  clip_grads<TG>(gv, grad_clip(a.gscale));
  if (a.have_state) {
    uint4 cm[F8_ELEMS / 16], cv[F8_ELEMS / 16];
    load_codes(qm, e0, nvalid, vec, cm);
    load_codes(qv, e0, nvalid, vec, cv);
    fp8_dequant_lane<FM, F8_ELEMS>(cm, fp8_dq<FM>(Fp8Meta{M.scale_m[grp], M.expand_m[grp], M.sqrt_minmax_m[grp]}),
                                   true, m);
    fp8_dequant_lane<FV, F8_ELEMS>(cv, fp8_dq<FV>(Fp8Meta{M.scale_v[grp], M.expand_v[grp], M.sqrt_minmax_v[grp]}),
                                   false, v);
  } else {
#pragma unroll
    for (int k = 0; k < F8_ELEMS; ++k) m[k] = v[k] = 0.f;
  }
#pragma unroll
  for (int k = 0; k < F8_ELEMS; ++k) {
    if constexpr (FASTQ) adamw_elem_fast<TP, TS>(pv[k], gv[k], m[k], v[k], a);
    else adamw_elem<TP, TS>(pv[k], gv[k], m[k], v[k], a);
  }
  if (vec) {
#pragma unroll
    for (int h = 0; h < F8_ELEMS / 8; ++h) Vec8<TP>::store(p + e0 + 8 * h, pv + 8 * h);
  } else {
#pragma unroll
    for (int k = 0; k < F8_ELEMS; ++k)
      if (k < nvalid) TP::store(p, e0 + k, pv[k]);
  }
  uint4 c[F8_ELEMS / 16];
  const Fp8Meta nm = full ? fp8_quant_group<FM, F8_ELEMS, true>(m, F8_ELEMS, true, a.emin, c)
                          : fp8_quant_group<FM, F8_ELEMS, false>(m, nvalid, true, a.emin, c);
  store_codes(qm, e0, nvalid, vec, c);
  const Fp8Meta nv = full ? fp8_quant_group<FV, F8_ELEMS, true>(v, F8_ELEMS, false, a.emin, c)
                          : fp8_quant_group<FV, F8_ELEMS, false>(v, nvalid, false, a.emin, c);
  store_codes(qv, e0, nvalid, vec, c);
  if (sub == 0) {
    M.scale_m[grp] = nm.scale;
    M.expand_m[grp] = nm.expand;
    M.sqrt_minmax_m[grp] = nm.sqrt_minmax;
    M.scale_v[grp] = nv.scale;
    M.expand_v[grp] = nv.expand;
    M.sqrt_minmax_v[grp] = nv.sqrt_minmax;
  }
}

template <class FM, class FV, bool FASTQ>
static int launch_adamw_fp8_q(const AdamWArgs& a, int param_dtype, int grad_dtype, hipStream_t s) {
  const dim3 grid(unsigned((a.nchunks + F8_GPW - 1) / F8_GPW)), block(ADAM_NT);
  if (param_dtype == MMUON_BF16 && grad_dtype == MMUON_BF16) {
    if (a.have_state)
      hipLaunchKernelGGL((adamw_fp8_kernel<BF16T, BF16T, F32T, FM, FV, FASTQ>), grid, block, 0, s, a);
    else
      hipLaunchKernelGGL((adamw_fp8_kernel<BF16T, BF16T, BF16T, FM, FV, FASTQ>), grid, block, 0, s, a);
  } else if (param_dtype == MMUON_F32 && grad_dtype == MMUON_F32) {
    hipLaunchKernelGGL((adamw_fp8_kernel<F32T, F32T, F32T, FM, FV, FASTQ>), grid, block, 0, s, a);
  } else {
    return -1;
  }
  return 0;
}
// the two update forms are separate kernels: with both in one kernel behind a
// uniform branch the compiler kept 141 VGPRs live (three waves per SIMD), each
// alone needs 110
template <class FM, class FV>
static int launch_adamw_fp8_f(const AdamWArgs& a, int param_dtype, int grad_dtype, hipStream_t s) {
  return a.fast_quot ? launch_adamw_fp8_q<FM, FV, true>(a, param_dtype, grad_dtype, s)
                     : launch_adamw_fp8_q<FM, FV, false>(a, param_dtype, grad_dtype, s);
}

int launch_adamw_fp8(const AdamWArgs& a, int param_dtype, int grad_dtype, int m_dtype, int v_dtype, hipStream_t s) {
  if (a.nchunks <= 0) return 0;
  const bool m8 = m_dtype == MMUON_F8E4M3, m5 = m_dtype == MMUON_F8E5M2;
  const bool v8 = v_dtype == MMUON_F8E4M3, v5 = v_dtype == MMUON_F8E5M2;
  if (m8 && v8) return launch_adamw_fp8_f<E4M3, E4M3>(a, param_dtype, grad_dtype, s);
  if (m8 && v5) return launch_adamw_fp8_f<E4M3, E5M2>(a, param_dtype, grad_dtype, s);
  if (m5 && v8) return launch_adamw_fp8_f<E5M2, E4M3>(a, param_dtype, grad_dtype, s);
  if (m5 && v5) return launch_adamw_fp8_f<E5M2, E5M2>(a, param_dtype, grad_dtype, s);
  return -1;
}

}  // namespace mmuon
