// Newton-Schulz quintic as a chain of batched gfx950 MFMA GEMM stages.
//
// One Newton-Schulz iteration over a stack of N blocks X (m x n, m <= n):
//   SYRK : A = s^2 * X X^T                      (m x m, symmetric, K = n)
//   POLY : P = b A + c A A                      (m x m, symmetric, K = m)
//   PX   : X' = s * (a X + P X)                 (m x n, K = m)
//   PX_APPLY (last iteration): param += alpha * bf16(X') written straight into
//          the parameter blocks, un-transposed for tall blocks.
// s = 1/(||X0||_F + 1e-7) on the first iteration (the Frobenius normalisation
// folded into the products: (sX)(sX)^T = s^2 XX^T and a(sX) + P(sX) = s(aX + PX)),
// 1 afterwards.
//
// bf16 kernels: v_mfma_f32_32x32x16_bf16, fp32 accumulation, bf16 stage outputs.
// 256-thread workgroups (4 waves) compute a 256x256 output tile; each wave a
// 128x128 sub-tile (4x4 MFMA tiles, 256 accumulators).  K advances 64 at a
// time through double-buffered LDS.  SYRK/POLY compute only the upper-triangle
// tiles and write each tile and its mirror.  The X operand of PX is row-major
// with the contraction along rows; it is staged into LDS as loaded and read
// transposed with ds_read_b64_tr_b16.
#include "common.hpp"
#include "kernels.hpp"

namespace mmuon {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

constexpr int NT = 256;      // threads per workgroup
constexpr int BK = 64;       // K tile
constexpr int LDK = BK + 8;  // LDS row stride of K-contiguous tiles (144 B: conflict-free b128 reads)
constexpr int XPAD = 32;     // LDS row padding of the row-major X tile (row stride = 64 mod 256 B)

constexpr int BM = 256;      // output tile (both dims)
constexpr int WM = 128;      // wave sub-tile
constexpr int WN = 128;
constexpr int TM = WM / 32;
constexpr int TN = WN / 32;

// Workgroups are dispatched round-robin over the 8 XCDs.  Map workgroup w to
// (block, tile) so that every tile of one block lands on the same XCD (and its
// L2), and the tiles of a block are dispatched back to back.
__device__ __forceinline__ bool decode_tile(int tiles, int N, int& b, int& t) {
  const int w = blockIdx.x;
  const int xcd = w & 7, local = w >> 3;
  b = xcd + 8 * (local / tiles);
  t = local % tiles;
  return b < N;
}

__device__ __forceinline__ void sym_tile(int t, int nt, int& ti, int& tj) {
  int i = 0;
  while (t >= nt - i) {
    t -= nt - i;
    ++i;
  }
  ti = i;
  tj = i + t;
}

__device__ __forceinline__ bf16x8 lds_b128(const uint16_t* p) {
  return *reinterpret_cast<const bf16x8*>(p);
}

// Transposed 8-element fragment of a row-major [k][col] LDS tile for a 32-wide
// MFMA operand: lane l receives column (c0 + l%32), rows k0 + 8*(l/32) + [0,8).
// ds_read_b64_tr_b16 works on groups of 16 lanes: lane i addresses 4 elements
// of row i/4 at column 4*(i%4) of a 4x16 block and receives column i of it.
__device__ __forceinline__ bf16x8 lds_tr_frag(const uint16_t* tile, int ld, int k0, int c0,
                                              int lane) {
  const int l16 = lane & 15;
  const int krow = k0 + ((lane >> 5) << 3) + (l16 >> 2);
  const int col = c0 + (((lane >> 4) & 1) << 4) + ((l16 & 3) << 2);
  const uint16_t* p0 = tile + krow * ld + col;
  const uint16_t* p1 = p0 + 4 * ld;
  const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p0));
  const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p1));
  typedef short i16x8 __attribute__((ext_vector_type(8)));
  const i16x8 v = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  return __builtin_bit_cast(bf16x8, v);
}

__device__ __forceinline__ f32x16 mfma(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ uint2 pack4(const float v[4]) {
  uint2 r;
  r.x = uint32_t(f2bf(v[0])) | (uint32_t(f2bf(v[1])) << 16);
  r.y = uint32_t(f2bf(v[2])) | (uint32_t(f2bf(v[3])) << 16);
  return r;
}
__device__ __forceinline__ void unpack4(uint2 r, float v[4]) {
  v[0] = __uint_as_float(r.x << 16);
  v[1] = __uint_as_float(r.x & 0xffff0000u);
  v[2] = __uint_as_float(r.y << 16);
  v[3] = __uint_as_float(r.y & 0xffff0000u);
}

// ---------------------------------------------------------------------------
// SYRK / POLY: symmetric m x m outputs, both operands K-contiguous rows.
// ---------------------------------------------------------------------------
template <int STAGE>
__global__ __launch_bounds__(NT, 1) void ns_sym_bf16(NsArgs a) {
  constexpr int CPT = BM * (BK / 8) / NT;  // 16-B chunks per thread per operand
  __shared__ __attribute__((aligned(16))) uint16_t lds[2][2][BM * LDK];

  const int nt = a.mp / BM;
  const int tiles = nt * (nt + 1) / 2;
  int b, t;
  if (!decode_tile(tiles, a.N, b, t)) return;
  int ti, tj;
  sym_tile(t, nt, ti, tj);

  const uint16_t* src;
  int ld, K;
  if (STAGE == NS_SYRK) {
    src = static_cast<const uint16_t*>(a.x_in) + int64_t(b) * a.mp * a.np;
    ld = a.np;
    K = a.kx;
  } else {
    src = static_cast<const uint16_t*>(a.a_in) + int64_t(b) * a.mp * a.mp;
    ld = a.mp;
    K = a.mp;
  }
  const uint16_t* pa = src + int64_t(ti) * BM * ld;
  const uint16_t* pb = src + int64_t(tj) * BM * ld;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  uint4 ra[CPT], rb[CPT];
  auto gload = [&](int k0) {
#pragma unroll
    for (int q = 0; q < CPT; ++q) {
      const int c = tid + NT * q, row = c >> 3, kc = c & 7;
      ra[q] = *reinterpret_cast<const uint4*>(pa + int64_t(row) * ld + k0 + kc * 8);
      rb[q] = *reinterpret_cast<const uint4*>(pb + int64_t(row) * ld + k0 + kc * 8);
    }
  };
  auto lstore = [&](int buf) {
#pragma unroll
    for (int q = 0; q < CPT; ++q) {
      const int c = tid + NT * q, row = c >> 3, kc = c & 7;
      *reinterpret_cast<uint4*>(&lds[buf][0][row * LDK + kc * 8]) = ra[q];
      *reinterpret_cast<uint4*>(&lds[buf][1][row * LDK + kc * 8]) = rb[q];
    }
  };

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = f32x16{};

  gload(0);
  lstore(0);
  __syncthreads();
  const int KT = K / BK;
  for (int kt = 0; kt < KT; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < KT) gload((kt + 1) * BK);
    const uint16_t* sA = lds[cur][0];
    const uint16_t* sB = lds[cur][1];
#pragma unroll
    for (int kk = 0; kk < BK / 16; ++kk) {
      bf16x8 fa[TM], fb[TN];
      const int koff = kk * 16 + (lane >> 5) * 8;
#pragma unroll
      for (int i = 0; i < TM; ++i) fa[i] = lds_b128(sA + (wm * WM + i * 32 + (lane & 31)) * LDK + koff);
#pragma unroll
      for (int j = 0; j < TN; ++j) fb[j] = lds_b128(sB + (wn * WN + j * 32 + (lane & 31)) * LDK + koff);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = mfma(fa[i], fb[j], acc[i][j]);
    }
    if (kt + 1 < KT) lstore(cur ^ 1);
    __syncthreads();
  }

  // epilogue: D[i][j] in registers, lane holds column j and rows i..i+3.
  float s2 = 1.f;
  if (STAGE == NS_SYRK && a.scale != nullptr) {
    const float s = a.scale[b];
    s2 = s * s;
  }
  uint16_t* out = static_cast<uint16_t*>(a.out) + int64_t(b) * a.mp * a.mp;
  const uint16_t* ain = static_cast<const uint16_t*>(a.a_in) + int64_t(b) * a.mp * a.mp;
#pragma unroll
  for (int i = 0; i < TM; ++i) {
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int col = tj * BM + wn * WN + j * 32 + (lane & 31);
#pragma unroll
      for (int qg = 0; qg < 4; ++qg) {
        const int row = ti * BM + wm * WM + i * 32 + qg * 8 + (lane >> 5) * 4;
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = acc[i][j][qg * 4 + e];
        if (STAGE == NS_SYRK) {
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] *= s2;
        } else {
          // A is symmetric: A[row+e][col] = A[col][row+e], one 8-B load.
          float av[4];
          unpack4(*reinterpret_cast<const uint2*>(ain + int64_t(col) * a.mp + row), av);
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = fmaf(a.cc, v[e], a.cb * av[e]);
        }
        const uint2 h = pack4(v);
        *reinterpret_cast<uint2*>(out + int64_t(col) * a.mp + row) = h;  // mirror tile
        if (ti != tj) {
          out[int64_t(row + 0) * a.mp + col] = uint16_t(h.x & 0xffffu);
          out[int64_t(row + 1) * a.mp + col] = uint16_t(h.x >> 16);
          out[int64_t(row + 2) * a.mp + col] = uint16_t(h.y & 0xffffu);
          out[int64_t(row + 3) * a.mp + col] = uint16_t(h.y >> 16);
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// PX / PX_APPLY: X' = s (a X + P X), m x n output, K = m.
// SWAP = true : D[j][i] in registers (lane holds i, four consecutive j) -> row-major
//               8-B stores of X' (and of untransposed parameter rows).
// SWAP = false: D[i][j] (lane holds j, four consecutive i) -> the transposed
//               parameter layout of tall blocks, param[j][i..i+3].
// ---------------------------------------------------------------------------
constexpr int PBN = 256;                     // output tile along n
constexpr int LDX = PBN + XPAD;

template <int STAGE, bool SWAP, class TP>
__global__ __launch_bounds__(NT, 1) void ns_px_bf16(NsArgs a) {
  constexpr int CPT_P = BM * (BK / 8) / NT;
  constexpr int CPT_X = BK * (PBN / 8) / NT;
  __shared__ __attribute__((aligned(16))) uint16_t sp[2][BM * LDK];
  __shared__ __attribute__((aligned(16))) uint16_t sx[2][BK * LDX];

  const int tiles_j = a.np / PBN;
  const int tiles = (a.mp / BM) * tiles_j;
  int b, t;
  if (!decode_tile(tiles, a.N, b, t)) return;
  const int ti = t / tiles_j, tj = t % tiles_j;

  const uint16_t* P = static_cast<const uint16_t*>(a.a_in) + int64_t(b) * a.mp * a.mp +
                      int64_t(ti) * BM * a.mp;
  const uint16_t* X = static_cast<const uint16_t*>(a.x_in) + int64_t(b) * a.mp * a.np;
  const uint16_t* Xt = X + tj * PBN;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  uint4 rp[CPT_P], rx[CPT_X];
  auto gload = [&](int k0) {
#pragma unroll
    for (int q = 0; q < CPT_P; ++q) {
      const int c = tid + NT * q, row = c >> 3, kc = c & 7;
      rp[q] = *reinterpret_cast<const uint4*>(P + int64_t(row) * a.mp + k0 + kc * 8);
    }
#pragma unroll
    for (int q = 0; q < CPT_X; ++q) {
      const int c = tid + NT * q, row = c / (PBN / 8), cc = c % (PBN / 8);
      rx[q] = *reinterpret_cast<const uint4*>(Xt + int64_t(k0 + row) * a.np + cc * 8);
    }
  };
  auto lstore = [&](int buf) {
#pragma unroll
    for (int q = 0; q < CPT_P; ++q) {
      const int c = tid + NT * q, row = c >> 3, kc = c & 7;
      *reinterpret_cast<uint4*>(&sp[buf][row * LDK + kc * 8]) = rp[q];
    }
#pragma unroll
    for (int q = 0; q < CPT_X; ++q) {
      const int c = tid + NT * q, row = c / (PBN / 8), cc = c % (PBN / 8);
      *reinterpret_cast<uint4*>(&sx[buf][row * LDX + cc * 8]) = rx[q];
    }
  };

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = f32x16{};

  gload(0);
  lstore(0);
  __syncthreads();
  const int KT = a.mp / BK;
  for (int kt = 0; kt < KT; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < KT) gload((kt + 1) * BK);
    const uint16_t* sP = sp[cur];
    const uint16_t* sX = sx[cur];
#pragma unroll
    for (int kk = 0; kk < BK / 16; ++kk) {
      bf16x8 fp[TM], fx[TN];
      const int koff = kk * 16 + (lane >> 5) * 8;
#pragma unroll
      for (int i = 0; i < TM; ++i) fp[i] = lds_b128(sP + (wm * WM + i * 32 + (lane & 31)) * LDK + koff);
#pragma unroll
      for (int j = 0; j < TN; ++j) fx[j] = lds_tr_frag(sX, LDX, kk * 16, wn * WN + j * 32, lane);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = SWAP ? mfma(fx[j], fp[i], acc[i][j]) : mfma(fp[i], fx[j], acc[i][j]);
    }
    if (kt + 1 < KT) lstore(cur ^ 1);
    __syncthreads();
  }

  const float s = a.scale != nullptr ? a.scale[b] : 1.f;
  uint16_t* out = static_cast<uint16_t*>(a.out) + int64_t(b) * a.mp * a.np;
  typename TP::storage* prm = nullptr;
  if (STAGE == NS_PX_APPLY) prm = reinterpret_cast<typename TP::storage*>(a.blocks[b].param);

#pragma unroll
  for (int i = 0; i < TM; ++i) {
#pragma unroll
    for (int j = 0; j < TN; ++j) {
#pragma unroll
      for (int qg = 0; qg < 4; ++qg) {
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = acc[i][j][qg * 4 + e];
        if (SWAP) {
          // lane: row i (X' row), columns jj..jj+3
          const int row = ti * BM + wm * WM + i * 32 + (lane & 31);
          const int col = tj * PBN + wn * WN + j * 32 + qg * 8 + (lane >> 5) * 4;
          float xv[4];
          unpack4(*reinterpret_cast<const uint2*>(X + int64_t(row) * a.np + col), xv);
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = s * fmaf(a.ca, xv[e], v[e]);
          if (STAGE == NS_PX) {
            *reinterpret_cast<uint2*>(out + int64_t(row) * a.np + col) = pack4(v);
          } else if (row < a.m) {
            // untransposed block: param[row][col] (rows = m, cols = n)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              if (col + e < a.n) {
                const int64_t o = int64_t(row) * a.n + col + e;
                TP::store(prm, o, fmaf(a.alpha, rbf(v[e]), TP::load(prm, o)));
              }
            }
          }
        } else {
          // lane: column j (X' column), rows ii..ii+3
          const int col = tj * PBN + wn * WN + j * 32 + (lane & 31);
          const int row = ti * BM + wm * WM + i * 32 + qg * 8 + (lane >> 5) * 4;
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = s * fmaf(a.ca, bf2f(X[int64_t(row + e) * a.np + col]), v[e]);
          if (STAGE == NS_PX) {
#pragma unroll
            for (int e = 0; e < 4; ++e) out[int64_t(row + e) * a.np + col] = f2bf(v[e]);
          } else if (col < a.n) {
            // tall block stored (rows = n, cols = m): param[col][row + e]
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              if (row + e < a.m) {
                const int64_t o = int64_t(col) * a.m + row + e;
                TP::store(prm, o, fmaf(a.alpha, rbf(v[e]), TP::load(prm, o)));
              }
            }
          }
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// fp32 Newton-Schulz (the pretrain copy keeps the buffer dtype).  Plain FMA
// tiles: 64x64 outputs, 256 threads x (4x4), K tile 16.  All tiles computed.
// ---------------------------------------------------------------------------
constexpr int FB = 64;
constexpr int FK = 16;

template <int STAGE, class TP>
__global__ __launch_bounds__(256) void ns_f32(NsArgs a) {
  __shared__ float sa[FK][FB + 4];
  __shared__ float sb[FK][FB + 4];
  const int b = blockIdx.z;
  const int ti = blockIdx.y, tj = blockIdx.x;
  const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
  const float* X = static_cast<const float*>(a.x_in) + int64_t(b) * a.mp * a.np;
  const float* A = static_cast<const float*>(a.a_in) + int64_t(b) * a.mp * a.mp;
  int K;
  if (STAGE == NS_SYRK) K = a.kx;
  else K = a.mp;
  float acc[4][4] = {};
  for (int k0 = 0; k0 < K; k0 += FK) {
    // thread loads one element of each operand tile: 64 rows x 16 k = 1024 = 4 per thread
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int idx = threadIdx.x + 256 * q;
      const int r = idx >> 4, k = idx & 15;
      float va, vb;
      if (STAGE == NS_SYRK) {
        va = X[int64_t(ti * FB + r) * a.np + k0 + k];
        vb = X[int64_t(tj * FB + r) * a.np + k0 + k];
      } else if (STAGE == NS_POLY) {
        va = A[int64_t(ti * FB + r) * a.mp + k0 + k];
        vb = A[int64_t(tj * FB + r) * a.mp + k0 + k];
      } else {
        va = A[int64_t(ti * FB + r) * a.mp + k0 + k];
        // X[k][j] tile: 16 rows x 64 cols
        const int kr = idx >> 6, c = idx & 63;
        vb = X[int64_t(k0 + kr) * a.np + tj * FB + c];
        sb[kr][c] = vb;
      }
      sa[k][r] = va;
      if (STAGE != NS_PX && STAGE != NS_PX_APPLY) sb[k][r] = vb;
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < FK; ++k) {
      float av[4], bv[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        av[e] = sa[k][ty * 4 + e];
        bv[e] = sb[k][tx * 4 + e];
      }
#pragma unroll
      for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int f = 0; f < 4; ++f) acc[e][f] = fmaf(av[e], bv[f], acc[e][f]);
    }
    __syncthreads();
  }
  const float s = a.scale != nullptr ? a.scale[b] : 1.f;
  typename TP::storage* prm = nullptr;
  if (STAGE == NS_PX_APPLY) prm = reinterpret_cast<typename TP::storage*>(a.blocks[b].param);
#pragma unroll
  for (int e = 0; e < 4; ++e) {
#pragma unroll
    for (int f = 0; f < 4; ++f) {
      const int i = ti * FB + ty * 4 + e, j = tj * FB + tx * 4 + f;
      float v = acc[e][f];
      if (STAGE == NS_SYRK) {
        static_cast<float*>(a.out)[int64_t(b) * a.mp * a.mp + int64_t(i) * a.mp + j] = v * (s * s);
      } else if (STAGE == NS_POLY) {
        static_cast<float*>(a.out)[int64_t(b) * a.mp * a.mp + int64_t(i) * a.mp + j] =
            fmaf(a.cc, v, a.cb * A[int64_t(i) * a.mp + j]);
      } else {
        const float u = s * fmaf(a.ca, X[int64_t(i) * a.np + j], v);
        if (STAGE == NS_PX) {
          static_cast<float*>(a.out)[int64_t(b) * a.mp * a.np + int64_t(i) * a.np + j] = u;
        } else if (i < a.m && j < a.n) {
          const int64_t o = a.transposed ? int64_t(j) * a.m + i : int64_t(i) * a.n + j;
          TP::store(prm, o, fmaf(a.alpha, u, TP::load(prm, o)));
        }
      }
    }
  }
}

template <int STAGE, class TP>
void launch_bf16(const NsArgs& a, hipStream_t s) {
  int tiles;
  if (STAGE == NS_SYRK || STAGE == NS_POLY) {
    const int nt = a.mp / BM;
    tiles = nt * (nt + 1) / 2;
  } else {
    tiles = (a.mp / BM) * (a.np / PBN);
  }
  const int grid = 8 * ((a.N + 7) / 8) * tiles;
  if (STAGE == NS_SYRK || STAGE == NS_POLY) {
    hipLaunchKernelGGL((ns_sym_bf16<STAGE>), dim3(grid), dim3(NT), 0, s, a);
  } else if (STAGE == NS_PX || !a.transposed) {
    hipLaunchKernelGGL((ns_px_bf16<STAGE, true, TP>), dim3(grid), dim3(NT), 0, s, a);
  } else {
    hipLaunchKernelGGL((ns_px_bf16<STAGE, false, TP>), dim3(grid), dim3(NT), 0, s, a);
  }
}

template <int STAGE, class TP>
void launch_f32(const NsArgs& a, hipStream_t s) {
  const int cols = (STAGE == NS_SYRK || STAGE == NS_POLY) ? a.mp : a.np;
  const dim3 grid(cols / FB, a.mp / FB, a.N);
  hipLaunchKernelGGL((ns_f32<STAGE, TP>), grid, dim3(256), 0, s, a);
}

}  // namespace

int ns_tile_m(int ns_dtype) { return ns_dtype == MMUON_BF16 ? BM : FB; }
int ns_tile_n(int ns_dtype) { return ns_dtype == MMUON_BF16 ? PBN : FB; }
int ns_tile_k(int ns_dtype) { return ns_dtype == MMUON_BF16 ? BK : FK; }

int launch_ns_stage(const NsArgs& a, int stage, int ns_dtype, int param_dtype, hipStream_t s) {
  if (ns_dtype == MMUON_BF16) {
    switch (stage) {
      case NS_SYRK: launch_bf16<NS_SYRK, BF16T>(a, s); return 0;
      case NS_POLY: launch_bf16<NS_POLY, BF16T>(a, s); return 0;
      case NS_PX: launch_bf16<NS_PX, BF16T>(a, s); return 0;
      case NS_PX_APPLY:
        if (param_dtype == MMUON_BF16) launch_bf16<NS_PX_APPLY, BF16T>(a, s);
        else launch_bf16<NS_PX_APPLY, F32T>(a, s);
        return 0;
    }
  } else if (ns_dtype == MMUON_F32) {
    switch (stage) {
      case NS_SYRK: launch_f32<NS_SYRK, F32T>(a, s); return 0;
      case NS_POLY: launch_f32<NS_POLY, F32T>(a, s); return 0;
      case NS_PX: launch_f32<NS_PX, F32T>(a, s); return 0;
      case NS_PX_APPLY:
        if (param_dtype == MMUON_BF16) launch_f32<NS_PX_APPLY, BF16T>(a, s);
        else launch_f32<NS_PX_APPLY, F32T>(a, s);
        return 0;
    }
  }
  return -1;
}

}  // namespace mmuon
