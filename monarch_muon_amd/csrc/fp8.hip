// FP8 optimizer-state kernels: the stand-alone codec and the fused
// dequantize -> momentum -> stack/cast -> requantize pass of the FP8-state step.
#include "common.hpp"
#include "fp8codec.hpp"
#include "kernels.hpp"

namespace mmuon {

constexpr int F8_NT = 256;  // 4 waves = 4 groups per workgroup

// coat_state_muon.py:103-114: fp32 values -> codes + per-group metadata.
__global__ __launch_bounds__(F8_NT) void fp8_quantize_kernel(const float* v, uint8_t* q, float* sc,
                                                             float* ex, float* smm, int64_t numel,
                                                             int sgn) {
  const int64_t grp = int64_t(blockIdx.x) * (F8_NT / 64) + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int64_t i0 = grp * 128 + lane, i1 = i0 + 64;
  if (grp * 128 >= numel) return;
  const bool v0 = i0 < numel, v1 = i1 < numel;
  const float x0 = v0 ? v[i0] : 0.f, x1 = v1 ? v[i1] : 0.f;
  uint8_t c0, c1;
  const Fp8Meta md = fp8_quant_group(x0, x1, v0, v1, sgn != 0, c0, c1);
  if (v0) q[i0] = c0;
  if (v1) q[i1] = c1;
  if (lane == 0) {
    sc[grp] = md.scale;
    ex[grp] = md.expand;
    smm[grp] = md.sqrt_minmax;
  }
}

// coat_state_muon.py:94-100
__global__ __launch_bounds__(F8_NT) void fp8_dequantize_kernel(const uint8_t* q, const float* sc,
                                                               const float* ex, const float* smm,
                                                               float* out, int64_t numel, int sgn) {
  const int64_t i = int64_t(blockIdx.x) * F8_NT + threadIdx.x;
  if (i >= numel) return;
  const int64_t grp = i >> 7;
  out[i] = fp8_dequant(q[i], Fp8Meta{sc[grp], ex[grp], smm[grp]}, sgn != 0);
}

void launch_fp8_quantize(const float* v, uint8_t* q, float* sc, float* ex, float* smm,
                         int64_t numel, bool sgn, hipStream_t s) {
  const int64_t groups = (numel + 127) / 128;
  if (groups == 0) return;
  hipLaunchKernelGGL(fp8_quantize_kernel, dim3(unsigned((groups + 3) / 4)), dim3(F8_NT), 0, s, v, q,
                     sc, ex, smm, numel, int(sgn));
}

void launch_fp8_dequantize(const uint8_t* q, const float* sc, const float* ex, const float* smm,
                           float* out, int64_t numel, bool sgn, hipStream_t s) {
  if (numel == 0) return;
  hipLaunchKernelGGL(fp8_dequantize_kernel, dim3(unsigned((numel + F8_NT - 1) / F8_NT)),
                     dim3(F8_NT), 0, s, q, sc, ex, smm, out, numel, int(sgn));
}

// ---------------------------------------------------------------------------
// Fused FP8 momentum pass.  The reference dequantizes the momentum to fp32,
// runs the fp32 momentum update (buf*mu, +g), stacks/casts for Newton-Schulz,
// and requantizes the updated fp32 momentum after the step
// (coat_state_muon.py:126-139).  The momentum is not touched between its update
// and the requantization, so both happen here in one pass.
// ---------------------------------------------------------------------------
template <class TG, class TX>
__device__ __forceinline__ float fp8_momentum_elem(const uint8_t* q, const Fp8Meta& md, int64_t i,
                                                   const typename TG::storage* g, float mu,
                                                   int have_state) {
  const float old = have_state ? fp8_dequant(q[i], md, true) : 0.f;
  const float t = old * mu;
  return t + TG::load(g, i);
}

// One wave per 128-group of a block (groups may wrap rows).  TRANS: the block
// is tall (rows > cols) and X holds its transpose; the general fallback for
// tall blocks whose width is not a multiple of 128 (scattered X stores).
template <class TG, class TX, bool TRANS>
__global__ __launch_bounds__(F8_NT) void fp8_pack_rows_kernel(PackArgs a, const mmuon_block_fp8* meta,
                                                              int rows, int cols, int have_state) {
  __shared__ float red[F8_NT / 64];
  const int b = blockIdx.y;
  const int lane = threadIdx.x & 63;
  const int64_t gpb = int64_t(rows) * cols / 128;  // groups per block
  const int64_t grp = int64_t(blockIdx.x) * (F8_NT / 64) + (threadIdx.x >> 6);
  const mmuon_block_ref ref = a.blocks[b];
  const mmuon_block_fp8 md = meta[b];
  const auto* g = reinterpret_cast<const typename TG::storage*>(ref.grad);
  uint8_t* q = reinterpret_cast<uint8_t*>(ref.buf);
  auto* x = reinterpret_cast<typename TX::storage*>(a.x) + int64_t(b) * a.mp * a.np;
  float ss = 0.f;
  if (grp < gpb) {
    Fp8Meta m0{0.f, 0.f, 0.f};
    if (have_state) m0 = Fp8Meta{md.scale[grp], md.expand[grp], md.sqrt_minmax[grp]};
    float nv[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int64_t e = grp * 128 + lane + 64 * h;
      nv[h] = fp8_momentum_elem<TG, TX>(q, m0, e, g, a.mu, have_state);
      const float xv = TX::round(nv[h]);
      ss += xv * xv;
      const int64_t r = e / cols, c = e % cols;
      TX::store(x, TRANS ? TX::xoff(a.mp, a.np, c, r) : TX::xoff(a.mp, a.np, r, c), xv);
    }
    uint8_t c0, c1;
    const Fp8Meta nm = fp8_quant_group(nv[0], nv[1], true, true, true, c0, c1);
    q[grp * 128 + lane] = c0;
    q[grp * 128 + lane + 64] = c1;
    if (lane == 0) {
      md.scale[grp] = nm.scale;
      md.expand[grp] = nm.expand;
      md.sqrt_minmax[grp] = nm.sqrt_minmax;
    }
  }
  const float tot = block_sum<F8_NT>(ss, red);
  if (threadIdx.x == 0) a.partial[int64_t(b) * a.nparts + blockIdx.x] = tot;
}

// rows > cols (cols % 128 == 0): a workgroup owns 64 block rows x 128 block
// columns (64 groups, 16 per wave) and writes the transposed X tile through LDS.
template <class TG, class TX>
__global__ __launch_bounds__(F8_NT) void fp8_pack_cols_kernel(PackArgs a, const mmuon_block_fp8* meta,
                                                              int rows, int cols, int have_state) {
  __shared__ float tile[64][128 + 1];
  __shared__ float red[F8_NT / 64];
  const int b = blockIdx.y;
  const int tiles_c = cols / 128;
  const int r0 = (blockIdx.x / tiles_c) * 64, c0 = (blockIdx.x % tiles_c) * 128;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const mmuon_block_ref ref = a.blocks[b];
  const mmuon_block_fp8 md = meta[b];
  const auto* g = reinterpret_cast<const typename TG::storage*>(ref.grad);
  uint8_t* q = reinterpret_cast<uint8_t*>(ref.buf);
  auto* x = reinterpret_cast<typename TX::storage*>(a.x) + int64_t(b) * a.mp * a.np;
  for (int k = 0; k < 16; ++k) {
    const int rl = wave * 16 + k, r = r0 + rl;
    float nv[2] = {0.f, 0.f};
    if (r < rows) {
      const int64_t grp = (int64_t(r) * cols + c0) / 128;
      Fp8Meta m0{0.f, 0.f, 0.f};
      if (have_state) m0 = Fp8Meta{md.scale[grp], md.expand[grp], md.sqrt_minmax[grp]};
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int64_t e = int64_t(r) * cols + c0 + lane + 64 * h;
        nv[h] = fp8_momentum_elem<TG, TX>(q, m0, e, g, a.mu, have_state);
      }
      uint8_t cA, cB;
      const Fp8Meta nm = fp8_quant_group(nv[0], nv[1], true, true, true, cA, cB);
      q[grp * 128 + lane] = cA;
      q[grp * 128 + lane + 64] = cB;
      if (lane == 0) {
        md.scale[grp] = nm.scale;
        md.expand[grp] = nm.expand;
        md.sqrt_minmax[grp] = nm.sqrt_minmax;
      }
    }
    tile[rl][lane] = TX::round(nv[0]);
    tile[rl][lane + 64] = TX::round(nv[1]);
  }
  __syncthreads();
  // X[c][r0 .. r0+63] for c in [c0, c0+128): thread -> (c = t/2, 32 consecutive r)
  float ss = 0.f;
  {
    const int cl = threadIdx.x >> 1, half = (threadIdx.x & 1) * 32;
    for (int k = 0; k < 32; ++k) {
      const int rl = half + k, r = r0 + rl;
      const float v = tile[rl][cl];
      ss += v * v;
      if (r < a.np) TX::store(x, TX::xoff(a.mp, a.np, c0 + cl, r), v);
    }
  }
  const float tot = block_sum<F8_NT>(ss, red);
  if (threadIdx.x == 0) a.partial[int64_t(b) * a.nparts + blockIdx.x] = tot;
}

// Zero the padding of an X stack (rows [m, mp), columns [n, np)): the FP8 pack
// writes only the real region.
template <class TX>
__global__ __launch_bounds__(256) void zero_pads_kernel(void* xv, int m, int n, int mp, int np_) {
  auto* x = reinterpret_cast<typename TX::storage*>(xv) + int64_t(blockIdx.y) * mp * np_;
  const int64_t total = int64_t(mp) * np_;
  for (int64_t e = int64_t(blockIdx.x) * 256 + threadIdx.x; e < total; e += int64_t(gridDim.x) * 256) {
    const int i = int(e / np_), j = int(e % np_);
    if (i >= m || j >= n) TX::store(x, TX::xoff(mp, np_, i, j), 0.f);
  }
}

int fp8_pack_nparts(int rows, int cols, bool transposed) {
  if (transposed && cols % 128 == 0) return ((rows + 63) / 64) * (cols / 128);
  const int64_t gpb = int64_t(rows) * cols / 128;
  return int((gpb + 3) / 4);
}

int launch_fp8_pack(const PackArgs& a, const mmuon_block_fp8* meta, int rows, int cols,
                    int grad_dtype, int x_dtype, bool transposed, int have_state,
                    hipStream_t s) {
  const dim3 grid(a.nparts, a.N), block(F8_NT);
  if (a.mp > a.m || a.np > a.n) {
    const dim3 zg(64, a.N);
    if (x_dtype == MMUON_BF16) hipLaunchKernelGGL((zero_pads_kernel<BF16T>), zg, dim3(256), 0, s, a.x, a.m, a.n, a.mp, a.np);
    else hipLaunchKernelGGL((zero_pads_kernel<F32T>), zg, dim3(256), 0, s, a.x, a.m, a.n, a.mp, a.np);
  }
#define MMUON_F8_CASE(GD, XD, TG, TX)                                                          \
  if (grad_dtype == GD && x_dtype == XD) {                                                     \
    if (transposed && cols % 128 == 0)                                                         \
      hipLaunchKernelGGL((fp8_pack_cols_kernel<TG, TX>), grid, block, 0, s, a, meta, rows, cols, \
                         have_state);                                                          \
    else if (transposed)                                                                       \
      hipLaunchKernelGGL((fp8_pack_rows_kernel<TG, TX, true>), grid, block, 0, s, a, meta, rows, \
                         cols, have_state);                                                    \
    else                                                                                       \
      hipLaunchKernelGGL((fp8_pack_rows_kernel<TG, TX, false>), grid, block, 0, s, a, meta, rows, \
                         cols, have_state);                                                    \
    return 0;                                                                                  \
  }
  MMUON_F8_CASE(MMUON_BF16, MMUON_BF16, BF16T, BF16T)
  MMUON_F8_CASE(MMUON_F32, MMUON_BF16, F32T, BF16T)
  MMUON_F8_CASE(MMUON_BF16, MMUON_F32, BF16T, F32T)
  MMUON_F8_CASE(MMUON_F32, MMUON_F32, F32T, F32T)
#undef MMUON_F8_CASE
  return -1;
}

}  // namespace mmuon
