// FP8 optimizer-state kernels: the stand-alone codec and the fused
// dequantize -> momentum -> stack/cast -> requantize pass of the FP8-state step.
// Every kernel is instantiated for both state formats (e4m3fn, e5m2) and takes
// expand_min at run time.
#include "common.hpp"
#include "fp8codec.hpp"
#include "kernels.hpp"

namespace mmuon {

constexpr int F8_NT = 256;

// ---------------------------------------------------------------------------
// Stand-alone codec over one flat tensor (coat_state_muon.py:94-114): one
// group of 128 per QL lanes, QE consecutive elements per lane; the last group
// may be short (numel % 128 != 0): its missing elements are neither read nor
// written and take no part in the group's max / min.
// ---------------------------------------------------------------------------
constexpr int QE = 16, QL = 128 / QE;
constexpr int Q_GPW = F8_NT / QL;  // 128-groups per workgroup

// A lane's QE values / codes: 16-B vector accesses for a full, aligned lane.
__device__ __forceinline__ bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

template <class F>
__global__ __launch_bounds__(F8_NT) void fp8_quantize_kernel(const float* v, uint8_t* q, float* sc, float* ex,
                                                             float* smm, int64_t numel, int sgn, float emin) {
  const int64_t grp = int64_t(blockIdx.x) * Q_GPW + (threadIdx.x / QL);
  if (grp * 128 >= numel) return;  // a group's lanes leave together
  const int sub = threadIdx.x % QL;
  const int64_t e0 = grp * 128 + sub * QE;
  const int nvalid = int(max(int64_t(0), min(int64_t(QE), numel - e0)));
  const bool full = grp * 128 + 128 <= numel;  // uniform over the group's lanes
  const bool vec = full && aligned16(v) && aligned16(q);
  float x[QE];
  if (vec) {
#pragma unroll
    for (int h = 0; h < QE / 4; ++h) {
      const float4 f = reinterpret_cast<const float4*>(v + e0)[h];
      x[4 * h] = f.x; x[4 * h + 1] = f.y; x[4 * h + 2] = f.z; x[4 * h + 3] = f.w;
    }
  } else {
#pragma unroll
    for (int k = 0; k < QE; ++k) x[k] = k < nvalid ? v[e0 + k] : 0.f;
  }
  uint4 c[QE / 16];
  const Fp8Meta md = full ? fp8_quant_group<F, QE, true>(x, QE, sgn != 0, emin, c)
                          : fp8_quant_group<F, QE, false>(x, nvalid, sgn != 0, emin, c);
  if (vec) {
    *reinterpret_cast<uint4*>(q + e0) = c[0];
  } else {
    const uint32_t w[4] = {c[0].x, c[0].y, c[0].z, c[0].w};
#pragma unroll
    for (int k = 0; k < QE; ++k)
      if (k < nvalid) q[e0 + k] = uint8_t(w[k >> 2] >> (8 * (k & 3)));
  }
  if (sub == 0) {
    sc[grp] = md.scale;
    ex[grp] = md.expand;
    smm[grp] = md.sqrt_minmax;
  }
}

template <class F>
__global__ __launch_bounds__(F8_NT) void fp8_dequantize_kernel(const uint8_t* q, const float* sc, const float* ex,
                                                               const float* smm, float* out, int64_t numel, int sgn) {
  const int64_t grp = int64_t(blockIdx.x) * Q_GPW + (threadIdx.x / QL);
  if (grp * 128 >= numel) return;
  const int sub = threadIdx.x % QL;
  const int64_t e0 = grp * 128 + sub * QE;
  const int nvalid = int(max(int64_t(0), min(int64_t(QE), numel - e0)));
  const bool vec = nvalid == QE && aligned16(q) && aligned16(out);
  uint4 c[1];
  if (vec) {
    c[0] = *reinterpret_cast<const uint4*>(q + e0);
  } else {
    uint32_t w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int k = 0; k < QE; ++k)
      if (k < nvalid) w[k >> 2] |= uint32_t(q[e0 + k]) << (8 * (k & 3));
    c[0] = make_uint4(w[0], w[1], w[2], w[3]);
  }
  float o[QE];
  fp8_dequant_lane<F, QE>(c, fp8_dq<F>(Fp8Meta{sc[grp], ex[grp], smm[grp]}), sgn != 0, o);
  if (vec) {
#pragma unroll
    for (int h = 0; h < QE / 4; ++h)
      reinterpret_cast<float4*>(out + e0)[h] = make_float4(o[4 * h], o[4 * h + 1], o[4 * h + 2], o[4 * h + 3]);
  } else {
#pragma unroll
    for (int k = 0; k < QE; ++k)
      if (k < nvalid) out[e0 + k] = o[k];
  }
}

template <class F>
static void launch_quantize_t(const float* v, uint8_t* q, float* sc, float* ex, float* smm, int64_t numel, bool sgn,
                              float emin, hipStream_t s) {
  const int64_t groups = (numel + 127) / 128;
  hipLaunchKernelGGL((fp8_quantize_kernel<F>), dim3(unsigned((groups + Q_GPW - 1) / Q_GPW)), dim3(F8_NT), 0, s, v, q,
                     sc, ex, smm, numel, int(sgn), emin);
}

int launch_fp8_quantize(const float* v, uint8_t* q, float* sc, float* ex, float* smm, int64_t numel, bool sgn,
                        int fp8_dtype, float emin, hipStream_t s) {
  if (numel == 0) return 0;
  if (fp8_dtype == MMUON_F8E4M3) launch_quantize_t<E4M3>(v, q, sc, ex, smm, numel, sgn, emin, s);
  else if (fp8_dtype == MMUON_F8E5M2) launch_quantize_t<E5M2>(v, q, sc, ex, smm, numel, sgn, emin, s);
  else return -1;
  return 0;
}

int launch_fp8_dequantize(const uint8_t* q, const float* sc, const float* ex, const float* smm, float* out,
                          int64_t numel, bool sgn, int fp8_dtype, hipStream_t s) {
  if (numel == 0) return 0;
  const int64_t groups = (numel + 127) / 128;
  const dim3 grid(unsigned((groups + Q_GPW - 1) / Q_GPW));
  if (fp8_dtype == MMUON_F8E4M3)
    hipLaunchKernelGGL((fp8_dequantize_kernel<E4M3>), grid, dim3(F8_NT), 0, s, q, sc, ex, smm, out, numel, int(sgn));
  else if (fp8_dtype == MMUON_F8E5M2)
    hipLaunchKernelGGL((fp8_dequantize_kernel<E5M2>), grid, dim3(F8_NT), 0, s, q, sc, ex, smm, out, numel, int(sgn));
  else
    return -1;
  return 0;
}

// ---------------------------------------------------------------------------
// Fused FP8 momentum pass.  The reference dequantizes the momentum to fp32,
// runs the fp32 momentum update (buf*mu, +g), stacks/casts for Newton-Schulz,
// and requantizes the updated fp32 momentum after the step
// (coat_state_muon.py:126-139).  The momentum is not touched between its update
// and the requantization, so both happen here in one pass.  Blocks of
// rows * cols % 128 == 0 only: every 128-group of the flattened parameter then
// lies inside one block.
// ---------------------------------------------------------------------------
// The fused pack: one 128-group per PL lanes, PE consecutive elements per lane.
constexpr int PE = 32, PL = 128 / PE;
constexpr int P_GPW = F8_NT / PL;  // 128-groups per workgroup

// This lane's PE momentum values after the update: dequantized codes (zeros
// without state) * mu + g, each op rounded to fp32 as the reference's fp32
// foreach ops round.
template <class TG, class F>
__device__ __forceinline__ void fp8_momentum_lane(const uint8_t* q, const mmuon_block_fp8& md, int64_t grp,
                                                  int64_t e0, const typename TG::storage* g, GradClip clip,
                                                  float mu, int have_state, float (&nv)[PE]) {
  float old[PE];
  if (have_state) {
    uint4 c[PE / 16];
#pragma unroll
    for (int h = 0; h < PE / 16; ++h) c[h] = *reinterpret_cast<const uint4*>(q + e0 + 16 * h);
    fp8_dequant_lane<F, PE>(c, fp8_dq<F>(Fp8Meta{md.scale[grp], md.expand[grp], md.sqrt_minmax[grp]}), true, old);
  } else {
#pragma unroll
    for (int k = 0; k < PE; ++k) old[k] = 0.f;
  }
  float gv[PE];
#pragma unroll
  for (int h = 0; h < PE / 8; ++h) Vec8<TG>::load(g + e0 + 8 * h, gv + 8 * h);
  clip_grads<TG>(gv, clip);
#pragma unroll
  for (int k = 0; k < PE; ++k) {
    const float t = old[k] * mu;
    nv[k] = t + gv[k];
  }
}

template <class F>
__device__ __forceinline__ void fp8_store_group(uint8_t* q, const mmuon_block_fp8& md, int64_t grp, int64_t e0,
                                                const float (&nv)[PE], float emin) {
  uint4 c[PE / 16];
  const Fp8Meta nm = fp8_quant_group<F, PE, true>(nv, PE, true, emin, c);
#pragma unroll
  for (int h = 0; h < PE / 16; ++h) *reinterpret_cast<uint4*>(q + e0 + 16 * h) = c[h];
  if (threadIdx.x % PL == 0) {
    md.scale[grp] = nm.scale;
    md.expand[grp] = nm.expand;
    md.sqrt_minmax[grp] = nm.sqrt_minmax;
  }
}

// PE consecutive values of one X row inside one 32-column panel: rounded to
// the NS dtype, stored, and their squares summed.  bf16 X: each pair is
// rounded by one v_cvt_pk_bf16_f32 and stored as it comes out.
template <class TX>
__device__ __forceinline__ float store_x_run(typename TX::storage* dst, const float (&nv)[PE]) {
  float ss = 0.f;
  if constexpr (sizeof(typename TX::storage) == 2) {
    uint32_t w[PE / 2];
#pragma unroll
    for (int j = 0; j < PE / 2; ++j) {
      w[j] = f2bf2(nv[2 * j], nv[2 * j + 1]);
      const float lo = __uint_as_float(w[j] << 16), hi = __uint_as_float(w[j] & 0xffff0000u);
      ss = fmaf(lo, lo, ss);
      ss = fmaf(hi, hi, ss);
    }
#pragma unroll
    for (int h = 0; h < PE / 8; ++h)
      reinterpret_cast<uint4*>(dst)[h] = make_uint4(w[4 * h], w[4 * h + 1], w[4 * h + 2], w[4 * h + 3]);
  } else {
#pragma unroll
    for (int k = 0; k < PE; ++k) ss = fmaf(nv[k], nv[k], ss);
#pragma unroll
    for (int h = 0; h < PE / 8; ++h) Vec8<TX>::store(dst + 8 * h, nv + 8 * h);
  }
  return ss;
}

// PL lanes per 128-group of a block (groups may wrap rows), PE elements per
// lane.  TRANS: the block is tall (rows > cols) and X holds its transpose; the
// fallback for tall blocks whose width is not a multiple of 128 (scattered X
// stores).
template <class TG, class TX, bool TRANS, class F>
__global__ __launch_bounds__(F8_NT) void fp8_pack_rows_kernel(PackArgs a, const mmuon_block_fp8* meta, int rows,
                                                              int cols, int have_state, float emin) {
  __shared__ float red[F8_NT / 64];
  const int b = blockIdx.y;
  const int64_t gpb = int64_t(rows) * cols / 128;  // groups per block
  const int64_t grp = int64_t(blockIdx.x) * P_GPW + (threadIdx.x / PL);
  const mmuon_block_ref ref = a.blocks[b];
  const mmuon_block_fp8 md = meta[b];
  const auto* g = reinterpret_cast<const typename TG::storage*>(ref.grad);
  uint8_t* q = reinterpret_cast<uint8_t*>(ref.buf);
  auto* x = reinterpret_cast<typename TX::storage*>(a.x) + int64_t(b) * a.mp * a.np;
  float ss = 0.f;
  if (grp < gpb) {  // uniform over the group's lanes
    const int64_t e0 = grp * 128 + (threadIdx.x % PL) * PE;
    float nv[PE];
    fp8_momentum_lane<TG, F>(q, md, grp, e0, g, grad_clip(a.gscale), a.mu, have_state, nv);
    if (!TRANS && cols % PE == 0) {
      // PE elements of one row, inside one 32-column panel (a block is below
      // 2^31 elements)
      const uint32_t r = uint32_t(e0) / uint32_t(cols), c = uint32_t(e0) - r * uint32_t(cols);
      ss = store_x_run<TX>(x + TX::xoff(a.mp, a.np, r, c), nv);
    } else {
#pragma unroll
      for (int k = 0; k < PE; ++k) {
        const int64_t r = (e0 + k) / cols, c = (e0 + k) % cols;
        const float xv = TX::round(nv[k]);
        ss = fmaf(xv, xv, ss);
        TX::store(x, TRANS ? TX::xoff(a.mp, a.np, c, r) : TX::xoff(a.mp, a.np, r, c), xv);
      }
    }
    fp8_store_group<F>(q, md, grp, e0, nv, emin);
  }
  const float tot = block_sum<F8_NT>(ss, red);
  if (threadIdx.x == 0) a.partial[int64_t(b) * a.nparts + blockIdx.x] = tot;
}

// rows > cols, cols % 128 == 0: a workgroup owns F8T_ROWS block rows x 128
// block columns (one group per row) and writes the transposed X tile through
// LDS: X rows c0 .. c0+127, columns r0 .. r0+F8T_ROWS-1 (one 64-B panel row
// per thread and half).
constexpr int F8T_ROWS = P_GPW;
static_assert(F8T_ROWS == 64, "two X panels per tile");
template <class TG, class TX, class F>
__global__ __launch_bounds__(F8_NT) void fp8_pack_cols_kernel(PackArgs a, const mmuon_block_fp8* meta, int rows,
                                                              int cols, int have_state, float emin) {
  __shared__ float tile[F8T_ROWS][128 + 4];
  __shared__ float red[F8_NT / 64];
  const int b = blockIdx.y;
  const int tiles_c = cols / 128;
  const int r0 = (blockIdx.x / tiles_c) * F8T_ROWS, c0 = (blockIdx.x % tiles_c) * 128;
  const int sub = threadIdx.x % PL, rl = threadIdx.x / PL, r = r0 + rl;
  const mmuon_block_ref ref = a.blocks[b];
  const mmuon_block_fp8 md = meta[b];
  const auto* g = reinterpret_cast<const typename TG::storage*>(ref.grad);
  uint8_t* q = reinterpret_cast<uint8_t*>(ref.buf);
  auto* x = reinterpret_cast<typename TX::storage*>(a.x) + int64_t(b) * a.mp * a.np;
  float nv[PE];
#pragma unroll
  for (int k = 0; k < PE; ++k) nv[k] = 0.f;
  if (r < rows) {  // uniform over the group's lanes
    const int64_t e0 = int64_t(r) * cols + c0 + sub * PE;
    const int64_t grp = e0 >> 7;
    fp8_momentum_lane<TG, F>(q, md, grp, e0, g, grad_clip(a.gscale), a.mu, have_state, nv);
    fp8_store_group<F>(q, md, grp, e0, nv, emin);
  }
#pragma unroll
  for (int k = 0; k < PE; k += 4) {
    float4* t4 = reinterpret_cast<float4*>(&tile[rl][sub * PE + k]);
    *t4 = make_float4(TX::round(nv[k]), TX::round(nv[k + 1]), TX::round(nv[k + 2]), TX::round(nv[k + 3]));
  }
  __syncthreads();
  // X row c0 + t/2, columns r0 + 32 (t%2) .. +31 (padding columns hold zeros)
  float ss = 0.f;
  {
    const int cl = threadIdx.x >> 1, half = (threadIdx.x & 1) * 32;
#pragma unroll
    for (int h = 0; h < 4; ++h) {
      float v[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        v[k] = tile[half + h * 8 + k][cl];
        ss = fmaf(v[k], v[k], ss);
      }
      if (r0 + half + h * 8 < a.np) Vec8<TX>::store(x + TX::xoff(a.mp, a.np, c0 + cl, r0 + half + h * 8), v);
    }
  }
  const float tot = block_sum<F8_NT>(ss, red);
  if (threadIdx.x == 0) a.partial[int64_t(b) * a.nparts + blockIdx.x] = tot;
}

// Zero the padding of an X stack (rows [m, mp), columns [n, np)): the FP8 pack
// writes only the real region, and runs after this kernel.  Walks 8-column
// chunks of the padding only: columns [n8, np) of every row (n8 = n rounded
// down to 8; the real elements of a straddling chunk are rewritten by the pack),
// then columns [0, n8) of rows [m, mp).  A chunk is 16 contiguous bytes in the
// bf16 panel layout and 32 in the fp32 row-major one.
template <class TX>
__global__ __launch_bounds__(256) void zero_pads_kernel(void* xv, int m, int n, int mp, int np_) {
  auto* x = reinterpret_cast<typename TX::storage*>(xv) + int64_t(blockIdx.y) * mp * np_;
  const int n8 = n & ~7;
  const int cr = (np_ - n8) >> 3;                  // right-pad chunks per row
  const int64_t right = int64_t(mp) * cr;
  const int64_t total = right + int64_t(mp - m) * (n8 >> 3);
  const float z[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int64_t c = int64_t(blockIdx.x) * 256 + threadIdx.x; c < total; c += int64_t(gridDim.x) * 256) {
    int i, j;
    if (c < right) {
      i = int(c / cr);
      j = n8 + 8 * int(c - int64_t(i) * cr);
    } else {
      const int64_t d = c - right;
      const int w = n8 >> 3;
      i = m + int(d / w);
      j = 8 * int(d - int64_t(i - m) * w);
    }
    Vec8<TX>::store(x + TX::xoff(mp, np_, i, j), z);
  }
}

int fp8_pack_nparts(int rows, int cols, bool transposed) {
  if (transposed && cols % 128 == 0) return ((rows + F8T_ROWS - 1) / F8T_ROWS) * (cols / 128);
  const int64_t gpb = int64_t(rows) * cols / 128;
  return int((gpb + P_GPW - 1) / P_GPW);
}

template <class TG, class TX, class F>
static void launch_fp8_pack_t(const PackArgs& a, const mmuon_block_fp8* meta, int rows, int cols, bool transposed,
                              int have_state, float emin, hipStream_t s) {
  const dim3 grid(a.nparts, a.N), block(F8_NT);
  if (transposed && cols % 128 == 0)
    hipLaunchKernelGGL((fp8_pack_cols_kernel<TG, TX, F>), grid, block, 0, s, a, meta, rows, cols, have_state, emin);
  else if (transposed)
    hipLaunchKernelGGL((fp8_pack_rows_kernel<TG, TX, true, F>), grid, block, 0, s, a, meta, rows, cols, have_state,
                       emin);
  else
    hipLaunchKernelGGL((fp8_pack_rows_kernel<TG, TX, false, F>), grid, block, 0, s, a, meta, rows, cols, have_state,
                       emin);
}

template <class F>
static int launch_fp8_pack_f(const PackArgs& a, const mmuon_block_fp8* meta, int rows, int cols, int grad_dtype,
                             int x_dtype, bool transposed, int have_state, float emin, hipStream_t s) {
#define MMUON_F8_CASE(GD, XD, TG, TX)                                                            \
  if (grad_dtype == GD && x_dtype == XD) {                                                       \
    launch_fp8_pack_t<TG, TX, F>(a, meta, rows, cols, transposed, have_state, emin, s);         \
    return 0;                                                                                    \
  }
  MMUON_F8_CASE(MMUON_BF16, MMUON_BF16, BF16T, BF16T)
  MMUON_F8_CASE(MMUON_F32, MMUON_BF16, F32T, BF16T)
  MMUON_F8_CASE(MMUON_BF16, MMUON_F32, BF16T, F32T)
  MMUON_F8_CASE(MMUON_F32, MMUON_F32, F32T, F32T)
#undef MMUON_F8_CASE
  return -1;
}

int launch_fp8_pack(const PackArgs& a, const mmuon_block_fp8* meta, int rows, int cols, int grad_dtype, int x_dtype,
                    int fp8_dtype, bool transposed, int have_state, float emin, hipStream_t s) {
  if ((grad_dtype != MMUON_BF16 && grad_dtype != MMUON_F32) || (x_dtype != MMUON_BF16 && x_dtype != MMUON_F32) ||
      (fp8_dtype != MMUON_F8E4M3 && fp8_dtype != MMUON_F8E5M2))
    return -1;
  if (a.mp > a.m || a.np > a.n) {
    const dim3 zg(16, a.N);
    if (x_dtype == MMUON_BF16) hipLaunchKernelGGL((zero_pads_kernel<BF16T>), zg, dim3(256), 0, s, a.x, a.m, a.n, a.mp, a.np);
    else hipLaunchKernelGGL((zero_pads_kernel<F32T>), zg, dim3(256), 0, s, a.x, a.m, a.n, a.mp, a.np);
  }
  if (fp8_dtype == MMUON_F8E4M3)
    return launch_fp8_pack_f<E4M3>(a, meta, rows, cols, grad_dtype, x_dtype, transposed, have_state, emin, s);
  return launch_fp8_pack_f<E5M2>(a, meta, rows, cols, grad_dtype, x_dtype, transposed, have_state, emin, s);
}

}  // namespace mmuon
