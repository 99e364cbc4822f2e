// Fused heavy-ball momentum + stack + cast + per-block sum of squares.
//
// One pass over a same-shape group of Monarch blocks:
//   buf <- round_B(round_B(buf * mu) + g)        (two torch ops, two roundings)
//   X   <- round_X(buf)  in Newton-Schulz orientation (transposed if rows>cols)
//   partial[b][wg] <- sum of X^2 over this workgroup's share of block b
// Algorithmic HBM traffic per element (fp32 momentum, bf16 grad, bf16 X):
// read g 2 B + read buf 4 B + write buf 4 B + write X 2 B = 12 B.
#include "common.hpp"
#include "kernels.hpp"

namespace mmuon {

template <class TB>
__device__ __forceinline__ float momentum_update(float buf, float g, float mu) {
  // compiled with -ffp-contract=off: the product is rounded before the sum,
  // as torch's separate mul_ and add_ do.
  const float t = TB::round(buf * mu);
  return TB::round(t + g);
}

constexpr int PACK_NT = 256;
constexpr int PACK_ITERS = 4;
constexpr int PACK_ELEMS = PACK_NT * 8 * PACK_ITERS;  // X elements per workgroup (row layout)

// rows <= cols: X[b][i][j] = buf[b][i][j], 8 elements per thread.
// fp32 X: the padded [mp][np] extent is walked in row-major order.
// bf16 X (32-column panels; mp, np multiples of 256): a workgroup owns 32 rows x
// 256 columns, and per iteration a wave covers 8 rows x 64 columns, so every
// wave reads whole 128-B lines of the momentum and gradient rows and writes two
// contiguous 512-B panel runs.
template <class TG, class TB, class TX>
__global__ __launch_bounds__(PACK_NT) void pack_rows_kernel(PackArgs a) {
  __shared__ float red[PACK_NT / 64];
  constexpr bool PANELS = sizeof(typename TX::storage) == 2;
  const int b = blockIdx.y;
  const mmuon_block_ref ref = a.blocks[b];
  const auto* g = reinterpret_cast<const typename TG::storage*>(ref.grad);
  auto* buf = reinterpret_cast<typename TB::storage*>(ref.buf);
  auto* x = reinterpret_cast<typename TX::storage*>(a.x) + int64_t(b) * a.mp * a.np;
  const int64_t total = int64_t(a.mp) * a.np;
  const int tiles_j = a.np / 256;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const GradClip clip = grad_clip(a.gscale);
  float ss = 0.f;
  if constexpr (PANELS) {
    const int i = (blockIdx.x / tiles_j) * 32 + wave * 8 + (lane >> 3);
    const int j0 = (blockIdx.x % tiles_j) * 256 + (lane & 7) * 8;
    if (a.vec && (blockIdx.x / tiles_j) * 32 + 32 <= a.m && (blockIdx.x % tiles_j) * 256 + 256 <= a.n) {
      // whole tile inside the block: every load of the thread is issued before
      // the first store, so the loads overlap instead of waiting one by one
      float gv[PACK_ITERS][8], bv[PACK_ITERS][8];
      const int64_t s0 = int64_t(i) * a.n + j0;
#pragma unroll
      for (int it = 0; it < PACK_ITERS; ++it) {
        Vec8<TG>::load(g + s0 + it * 64, gv[it]);
        Vec8<TB>::load(buf + s0 + it * 64, bv[it]);
      }
#pragma unroll
      for (int it = 0; it < PACK_ITERS; ++it) {
        float v[8];
        clip_grads<TG>(gv[it], clip);
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          bv[it][q] = momentum_update<TB>(bv[it][q], gv[it][q], a.mu);
          v[q] = TX::round(bv[it][q]);
          ss += v[q] * v[q];
        }
        // streaming stores (each line written once by this pass)
        Vec8<TB>::store_nt(buf + s0 + it * 64, bv[it]);
        Vec8<TX>::store_nt(x + TX::xoff(a.mp, a.np, i, j0 + it * 64), v);
      }
      const float tot = block_sum<PACK_NT>(ss, red);
      if (threadIdx.x == 0) a.partial[int64_t(b) * a.nparts + blockIdx.x] = tot;
      return;
    }
  }
#pragma unroll
  for (int it = 0; it < PACK_ITERS; ++it) {
    int i, j;
    if constexpr (PANELS) {
      i = (blockIdx.x / tiles_j) * 32 + wave * 8 + (lane >> 3);
      j = (blockIdx.x % tiles_j) * 256 + it * 64 + (lane & 7) * 8;
    } else {
      const int64_t e = int64_t(blockIdx.x) * PACK_ELEMS + (int64_t(it) * PACK_NT + threadIdx.x) * 8;
      if (e >= total) break;
      i = int(e / a.np);
      j = int(e % a.np);
    }
    float v[8];
    if (a.vec && i < a.m && j + 8 <= a.n) {
      const int64_t s = int64_t(i) * a.n + j;
      float gv[8], bv[8];
      Vec8<TG>::load(g + s, gv);
      Vec8<TB>::load(buf + s, bv);
      clip_grads<TG>(gv, clip);
#pragma unroll
      for (int q = 0; q < 8; ++q) bv[q] = momentum_update<TB>(bv[q], gv[q], a.mu);
      Vec8<TB>::store(buf + s, bv);
#pragma unroll
      for (int q = 0; q < 8; ++q) v[q] = TX::round(bv[q]);
    } else {
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        v[q] = 0.f;
        if (i < a.m && j + q < a.n) {
          const int64_t s = int64_t(i) * a.n + j + q;
          const float nb = momentum_update<TB>(TB::load(buf, s), clipped<TG>(TG::load(g, s), clip), a.mu);
          TB::store(buf, s, nb);
          v[q] = TX::round(nb);
        }
      }
    }
#pragma unroll
    for (int q = 0; q < 8; ++q) ss += v[q] * v[q];
    Vec8<TX>::store(x + TX::xoff(a.mp, a.np, i, j), v);  // 8 elements stay in one panel
  }
  const float tot = block_sum<PACK_NT>(ss, red);
  if (threadIdx.x == 0) a.partial[int64_t(b) * a.nparts + blockIdx.x] = tot;
}

// rows > cols: X[b][i][j] = buf[b][j][i].  A workgroup owns 32 buf rows (one
// 32-column panel of X) x 256 buf columns (256 X rows): phase 1 reads the 32
// rows (every wave two contiguous 1 KiB fp32 row segments per load), updates
// the momentum and stages the rounded values in LDS; phase 2 gives each thread
// one X row of the panel (64 contiguous bytes for bf16 X), so the workgroup's
// X writes are one contiguous 16 KiB run.
constexpr int PCOL_ROWS = 32;   // buf rows per workgroup
constexpr int PCOL_COLS = 256;  // buf columns per workgroup (= PACK_NT)
static_assert(PCOL_COLS == PACK_NT, "one X row per thread in phase 2");
template <class TG, class TB, class TX>
__global__ __launch_bounds__(PACK_NT) void pack_cols_kernel(PackArgs a) {
  __shared__ float tile[PCOL_ROWS][PCOL_COLS + 4];
  __shared__ float red[PACK_NT / 64];
  constexpr int CHUNKS = PCOL_ROWS * PCOL_COLS / 8 / PACK_NT;  // 8-element chunks per thread
  const int b = blockIdx.y;
  const int tiles_i = (a.mp + PCOL_COLS - 1) / PCOL_COLS;  // the last one partial when mp % 256 != 0
  const int tj = blockIdx.x / tiles_i, ti = blockIdx.x % tiles_i;
  const int r0 = tj * PCOL_ROWS, c0 = ti * PCOL_COLS;  // buf rows (X columns), buf columns (X rows)
  const mmuon_block_ref ref = a.blocks[b];
  const auto* g = reinterpret_cast<const typename TG::storage*>(ref.grad);
  auto* buf = reinterpret_cast<typename TB::storage*>(ref.buf);
  auto* x = reinterpret_cast<typename TX::storage*>(a.x) + int64_t(b) * a.mp * a.np;
  const GradClip clip = grad_clip(a.gscale);
  float ss = 0.f;
  // phase 1: chunk e = q * PACK_NT + t covers buf row r0 + e/32, columns c0 + 8 (e%32) + [0, 8)
  if (a.vec && r0 + PCOL_ROWS <= a.n && c0 + PCOL_COLS <= a.m) {
    float gv[CHUNKS][8], bv[CHUNKS][8];
#pragma unroll
    for (int q = 0; q < CHUNKS; ++q) {
      const int e = q * PACK_NT + threadIdx.x;
      const int64_t s = int64_t(r0 + (e >> 5)) * a.m + c0 + (e & 31) * 8;
      Vec8<TG>::load(g + s, gv[q]);
      Vec8<TB>::load(buf + s, bv[q]);
    }
    if (clip.on) {
#pragma unroll
      for (int q = 0; q < CHUNKS; ++q) clip_grads<TG>(gv[q], clip);
    }
#pragma unroll
    for (int q = 0; q < CHUNKS; ++q) {
      const int e = q * PACK_NT + threadIdx.x;
      const int64_t s = int64_t(r0 + (e >> 5)) * a.m + c0 + (e & 31) * 8;
      float v[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        bv[q][k] = momentum_update<TB>(bv[q][k], gv[q][k], a.mu);
        v[k] = TX::round(bv[q][k]);
        ss += v[k] * v[k];
      }
      Vec8<TB>::store(buf + s, bv[q]);
      float4* t4 = reinterpret_cast<float4*>(&tile[e >> 5][(e & 31) * 8]);
      t4[0] = make_float4(v[0], v[1], v[2], v[3]);
      t4[1] = make_float4(v[4], v[5], v[6], v[7]);
    }
  } else {
#pragma unroll
    for (int q = 0; q < CHUNKS; ++q) {
      const int e = q * PACK_NT + threadIdx.x;
      const int r = r0 + (e >> 5), c = c0 + (e & 31) * 8;
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        float v = 0.f;
        if (r < a.n && c + k < a.m) {
          const int64_t s = int64_t(r) * a.m + c + k;
          const float nb = momentum_update<TB>(TB::load(buf, s), clipped<TG>(TG::load(g, s), clip), a.mu);
          TB::store(buf, s, nb);
          v = TX::round(nb);
        }
        ss += v * v;
        tile[e >> 5][(e & 31) * 8 + k] = v;
      }
    }
  }
  __syncthreads();
  // phase 2: X row c0 + t, columns r0 .. r0+31 (zeros in the padding)
  const int t = threadIdx.x;
  if (c0 + t < a.mp) {
#pragma unroll
    for (int h = 0; h < PCOL_ROWS / 8; ++h) {
      float v[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) v[k] = tile[h * 8 + k][t];
      Vec8<TX>::store(x + TX::xoff(a.mp, a.np, c0 + t, r0 + h * 8), v);
    }
  }
  const float tot = block_sum<PACK_NT>(ss, red);
  if (threadIdx.x == 0) a.partial[int64_t(b) * a.nparts + blockIdx.x] = tot;
}

int pack_nparts(int mp, int np_, bool transposed) {
  if (transposed) return ((mp + PCOL_COLS - 1) / PCOL_COLS) * (np_ / PCOL_ROWS);
  const int64_t total = int64_t(mp) * np_;
  return int((total + PACK_ELEMS - 1) / PACK_ELEMS);
}

template <class TG, class TB, class TX>
static void launch_pack_t(const PackArgs& a, bool transposed, hipStream_t s) {
  const dim3 grid(a.nparts, a.N);
  if (transposed)
    hipLaunchKernelGGL((pack_cols_kernel<TG, TB, TX>), grid, dim3(PACK_NT), 0, s, a);
  else
    hipLaunchKernelGGL((pack_rows_kernel<TG, TB, TX>), grid, dim3(PACK_NT), 0, s, a);
}

int launch_pack(const PackArgs& a, int grad_dtype, int buf_dtype, int x_dtype, bool transposed,
                hipStream_t s) {
#define MMUON_PACK_CASE(GD, BD, XD, TG, TB, TX)                         \
  if (grad_dtype == GD && buf_dtype == BD && x_dtype == XD) {           \
    launch_pack_t<TG, TB, TX>(a, transposed, s);                        \
    return 0;                                                           \
  }
  MMUON_PACK_CASE(MMUON_BF16, MMUON_F32, MMUON_BF16, BF16T, F32T, BF16T)
  MMUON_PACK_CASE(MMUON_BF16, MMUON_BF16, MMUON_BF16, BF16T, BF16T, BF16T)
  MMUON_PACK_CASE(MMUON_F32, MMUON_F32, MMUON_BF16, F32T, F32T, BF16T)
  MMUON_PACK_CASE(MMUON_F32, MMUON_BF16, MMUON_BF16, F32T, BF16T, BF16T)
  MMUON_PACK_CASE(MMUON_F32, MMUON_F32, MMUON_F32, F32T, F32T, F32T)
  MMUON_PACK_CASE(MMUON_BF16, MMUON_F32, MMUON_F32, BF16T, F32T, F32T)
  MMUON_PACK_CASE(MMUON_BF16, MMUON_BF16, MMUON_F32, BF16T, BF16T, F32T)
  MMUON_PACK_CASE(MMUON_F32, MMUON_BF16, MMUON_F32, F32T, BF16T, F32T)
#undef MMUON_PACK_CASE
  return -1;
}

// ---------------------------------------------------------------------------
// Per-block normalisation factor s = 1 / (||X||_F + 1e-7), from the partial sums.
// bf16 Newton-Schulz: the reference computes the norm of the bf16 stack as a
// bf16 tensor and adds 1e-7 in bf16 (membench monarch_muon.py:38-39), so both
// roundings are applied here; fp32: plain fp32.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(64) void block_scale_kernel(const float* partial, int nparts,
                                                         float* scale, int bf16_norm) {
  const int b = blockIdx.x;
  float s = 0.f;
  for (int k = threadIdx.x; k < nparts; k += 64) s += partial[int64_t(b) * nparts + k];
  s = wave_sum(s);
  if (threadIdx.x == 0) {
    float nrm = sqrtf(s);
    float d = bf16_norm ? rbf(rbf(nrm) + 1e-7f) : nrm + 1e-7f;
    scale[b] = 1.0f / d;
  }
}

void launch_block_scale(const float* partial, int nparts, float* scale, int N, bool bf16_norm,
                        hipStream_t s) {
  hipLaunchKernelGGL(block_scale_kernel, dim3(N), dim3(64), 0, s, partial, nparts, scale,
                     bf16_norm ? 1 : 0);
}

}  // namespace mmuon
