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
// 128x128 sub-tile (4x4 MFMA tiles, 256 accumulators in AGPRs).  K advances 32
// at a time through a 4-slot LDS ring filled by direct global->LDS loads
// (global_load_lds_dwordx4), three slices in flight ahead of the one in use.
// SYRK/POLY compute only the upper-triangle tiles and write each tile and its
// mirror.  The X operand of PX is row-major with the contraction along rows; it
// is staged into LDS as loaded and read transposed with ds_read_b64_tr_b16.
#include "common.hpp"
#include "kernels.hpp"

namespace mmuon {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

constexpr int NT = 256;      // threads per workgroup (4 waves, 2 x 2)
constexpr int BK = 32;       // K slice per pipeline stage
constexpr int NSTAGE = 4;    // LDS ring depth (three slices in flight ahead of the one in use)
constexpr int BM = 256;      // output tile, both dimensions
constexpr int WM = 128;      // wave sub-tile
constexpr int TM = WM / 32;  // 32x32 MFMA tiles per wave and dimension
constexpr int SLICE = 256 * BK;        // elements of one operand slice (16 KiB)
constexpr int DMA_PER_OPERAND = SLICE * 2 / (NT * 16);  // 16-B direct loads per thread per slice

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

// Wait until at most N direct-to-LDS loads of this thread are outstanding
// (vector-memory loads complete in issue order).
template <int N>
__device__ __forceinline__ void wait_vm() {
  if constexpr (N == 0) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  else if constexpr (N == 8) asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
  else asm volatile("s_waitcnt vmcnt(16)" ::: "memory");
}

typedef __attribute__((address_space(3))) void lds_void;

// 16-B direct global->LDS load: lane l of the wave lands at lds_base + 16*l
// (M0 holds the wave-uniform LDS base).  Issued as inline assembly so that the
// compiler's wait-count pass does not guard every later LDS read with a
// vmcnt(0); the pipeline waits for exactly the slice it reads (wait_vm, in-order
// completion of vector-memory loads) and then synchronises the workgroup.
__device__ __forceinline__ void dma16(const uint16_t* g, uint16_t* lds_base) {
  const uint32_t m0 = uint32_t(reinterpret_cast<uintptr_t>((lds_void*)lds_base));
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
               :
               : "v"(g), "s"(__builtin_amdgcn_readfirstlane(m0))
               : "memory");
}

// Workgroup barrier that also stops the compiler from moving LDS reads above it.
__device__ __forceinline__ void barrier() {
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// ----- LDS layouts --------------------------------------------------------
// K-major slice [256 rows][32 k]: a row is four 16-B chunks; chunk c of row r
// sits in slot c ^ ((r >> 2) & 3), so the 16 rows read by one quarter-wave's
// ds_read_b128 cover all 64 banks.
// Row-major X slice [32 k][256 cols]: a row is eight 64-B granules; granule g
// of row k sits at g ^ (k & 3), so the four rows a ds_read_b64_tr_b16 group
// touches land on distinct bank quarters.

// Issue one K-major operand slice: 256 rows of 32 k starting at `src` (row
// stride ld elements, k offset already applied).  Wave w, instruction q covers
// rows 16*(4w+q) .. +15; lane l loads row l/4, chunk (l%4) ^ ((l>>4)&3).
__device__ __forceinline__ void issue_kmajor(const uint16_t* src, int64_t ld, uint16_t* slice,
                                             int wave, int lane) {
  const int r_in = lane >> 2;
  const int chunk = (lane & 3) ^ ((lane >> 4) & 3);
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int grp = wave * 4 + q;
    dma16(src + int64_t(grp * 16 + r_in) * ld + chunk * 8, slice + grp * 16 * BK);
  }
}

// Issue one row-major X slice: 32 rows of 256 columns at `src` (row stride ld).
// Wave w, instruction q covers rows 2*(4w+q) .. +1; lane l loads row l/32,
// physical chunk l%32 = logical granule ((l%32)/4) ^ (row & 3), chunk l%4.
__device__ __forceinline__ void issue_rowmajor(const uint16_t* src, int64_t ld, uint16_t* slice,
                                               int wave, int lane) {
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int grp = wave * 4 + q;
    const int row = grp * 2 + (lane >> 5);
    const int lg = ((lane & 31) >> 2) ^ (row & 3);
    dma16(src + int64_t(row) * ld + lg * 32 + (lane & 3) * 8, slice + grp * 2 * 256);
  }
}

// 8-element K-major fragment of a 32-row MFMA operand (rows r0 + lane%32,
// k = 16*kk + 8*(lane/32) + [0,8)).
__device__ __forceinline__ bf16x8 frag_kmajor(const uint16_t* slice, int r0, int kk, int lane) {
  const int r = r0 + (lane & 31);
  const int c = (kk * 2 + (lane >> 5)) ^ ((r >> 2) & 3);
  return *reinterpret_cast<const bf16x8*>(slice + r * BK + c * 8);
}

// Same fragment shape read transposed out of a row-major X slice: lane l
// receives column c0 + l%32, rows 16*kk + 8*(l/32) + [0,8).  ds_read_b64_tr_b16
// works on 16-lane groups: lane i addresses 4 elements of row i/4 at column
// 4*(i%4) of a 4x16 block and receives column i of that block.
__device__ __forceinline__ bf16x8 frag_rowmajor_tr(const uint16_t* slice, int c0, int kk, int lane) {
  const int l16 = lane & 15;
  const int col = c0 + (((lane >> 4) & 1) << 4) + ((l16 & 3) << 2);
  const int gran = col >> 5, within = col & 31;
  const int k0 = kk * 16 + ((lane >> 5) << 3) + (l16 >> 2);
  const int k1 = k0 + 4;
  const uint16_t* p0 = slice + k0 * 256 + ((gran ^ (k0 & 3)) << 5) + within;
  const uint16_t* p1 = slice + k1 * 256 + ((gran ^ (k1 & 3)) << 5) + within;
  const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p0));
  const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p1));
  typedef short i16x8 __attribute__((ext_vector_type(8)));
  const i16x8 v = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  return __builtin_bit_cast(bf16x8, v);
}

// ---------------------------------------------------------------------------
// The pipelined main loop shared by every stage.  ROWMAJOR_C: the column
// operand is the row-major X stack (PX stages), else K-major (SYRK/POLY).
// SWAP: D holds [col][row] (lane owns a row index and four consecutive column
// indices) instead of [row][col].
// ---------------------------------------------------------------------------
// Ring slots are distinct LDS objects so that the compiler's wait-count pass
// can tell the slices apart and wait only for the slice about to be read.
struct Ring {
  uint16_t* r0; uint16_t* r1; uint16_t* r2; uint16_t* r3;
  uint16_t* c0; uint16_t* c1; uint16_t* c2; uint16_t* c3;
  template <int S> __device__ __forceinline__ uint16_t* r() const {
    if constexpr (S == 0) return r0; else if constexpr (S == 1) return r1;
    else if constexpr (S == 2) return r2; else return r3;
  }
  template <int S> __device__ __forceinline__ uint16_t* c() const {
    if constexpr (S == 0) return c0; else if constexpr (S == 1) return c1;
    else if constexpr (S == 2) return c2; else return c3;
  }
};

template <bool ROWMAJOR_C, bool SWAP>
struct Pipe {
  const uint16_t* rsrc;
  int64_t rld;
  const uint16_t* csrc;
  int64_t cld;
  int KT;
  int wave, lane, wm, wn;

  template <int S>
  __device__ __forceinline__ void issue(const Ring& ring, int kt) const {
    issue_kmajor(rsrc + kt * BK, rld, ring.template r<S>(), wave, lane);
    if (ROWMAJOR_C) issue_rowmajor(csrc + int64_t(kt) * BK * cld, cld, ring.template c<S>(), wave, lane);
    else issue_kmajor(csrc + kt * BK, cld, ring.template c<S>(), wave, lane);
  }

  template <int S>
  __device__ __forceinline__ void compute(const Ring& ring, f32x16 (&acc)[TM][TM]) const {
    const uint16_t* sr = ring.template r<S>();
    const uint16_t* sc = ring.template c<S>();
    // every fragment of the slice first (both 16-deep k steps), then the MFMAs
    bf16x8 fr[BK / 16][TM], fc[BK / 16][TM];
#pragma unroll
    for (int kk = 0; kk < BK / 16; ++kk) {
#pragma unroll
      for (int j = 0; j < TM; ++j)
        fc[kk][j] = ROWMAJOR_C ? frag_rowmajor_tr(sc, wn * WM + j * 32, kk, lane)
                               : frag_kmajor(sc, wn * WM + j * 32, kk, lane);
#pragma unroll
      for (int i = 0; i < TM; ++i) fr[kk][i] = frag_kmajor(sr, wm * WM + i * 32, kk, lane);
    }
#pragma unroll
    for (int kk = 0; kk < BK / 16; ++kk)
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TM; ++j)
          acc[i][j] = SWAP ? mfma(fc[kk][j], fr[kk][i], acc[i][j]) : mfma(fr[kk][i], fc[kk][j], acc[i][j]);
  }

  // k-slice kt lives in ring slot S = kt % 4; slices kt+1, kt+2 are in flight.
  template <int S>
  __device__ __forceinline__ void step(const Ring& ring, int kt, f32x16 (&acc)[TM][TM]) const {
    if (kt >= KT) return;
    if (kt + 2 < KT) wait_vm<2 * 2 * DMA_PER_OPERAND>();
    else if (kt + 1 < KT) wait_vm<2 * DMA_PER_OPERAND>();
    else wait_vm<0>();
    barrier();
    if (kt + 3 < KT) issue<(S + 3) & 3>(ring, kt + 3);
    compute<S>(ring, acc);
  }

  __device__ __forceinline__ void run(const Ring& ring, f32x16 (&acc)[TM][TM]) const {
    issue<0>(ring, 0);
    if (KT > 1) issue<1>(ring, 1);
    if (KT > 2) issue<2>(ring, 2);
    for (int kt = 0; kt < KT; kt += 4) {
      step<0>(ring, kt, acc);
      step<1>(ring, kt + 1, acc);
      step<2>(ring, kt + 2, acc);
      step<3>(ring, kt + 3, acc);
    }
  }
};

template <bool ROWMAJOR_C, bool SWAP>
__device__ __forceinline__ void mainloop(const uint16_t* rsrc, int64_t rld, const uint16_t* csrc,
                                         int64_t cld, int KT, const Ring& ring, f32x16 (&acc)[TM][TM]) {
  Pipe<ROWMAJOR_C, SWAP> p;
  p.rsrc = rsrc;
  p.rld = rld;
  p.csrc = csrc;
  p.cld = cld;
  p.KT = KT;
  p.lane = threadIdx.x & 63;
  p.wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  p.wm = p.wave >> 1;
  p.wn = p.wave & 1;
  p.run(ring, acc);
}

#define MMUON_RING_DECL                                                                        \
  __shared__ __attribute__((aligned(1024))) uint16_t r0_[SLICE], r1_[SLICE], r2_[SLICE], r3_[SLICE]; \
  __shared__ __attribute__((aligned(1024))) uint16_t c0_[SLICE], c1_[SLICE], c2_[SLICE], c3_[SLICE]; \
  Ring ring;                                                                                   \
  ring.r0 = r0_; ring.r1 = r1_; ring.r2 = r2_; ring.r3 = r3_;                                  \
  ring.c0 = c0_; ring.c1 = c1_; ring.c2 = c2_; ring.c3 = c3_;

// ---------------------------------------------------------------------------
// SYRK / POLY: symmetric m x m outputs, both operands K-major rows.
// ---------------------------------------------------------------------------
template <int STAGE>
__global__ __launch_bounds__(NT, 1) void ns_sym_bf16(NsArgs a) {
  MMUON_RING_DECL

  const int nt = a.mp / BM;
  const int tiles = nt * (nt + 1) / 2;
  int b, t;
  if (!decode_tile(tiles, a.N, b, t)) return;
  int ti, tj;
  sym_tile(t, nt, ti, tj);

  const uint16_t* src;
  int64_t ld;
  int K;
  if (STAGE == NS_SYRK) {
    src = static_cast<const uint16_t*>(a.x_in) + int64_t(b) * a.mp * a.np;
    ld = a.np;
    K = a.kx;
  } else {
    src = static_cast<const uint16_t*>(a.a_in) + int64_t(b) * a.mp * a.mp;
    ld = a.mp;
    K = a.mp;
  }
  f32x16 acc[TM][TM];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TM; ++j) acc[i][j] = f32x16{};
  mainloop<false, false>(src + int64_t(ti) * BM * ld, ld, src + int64_t(tj) * BM * ld, ld, K / BK, ring, acc);

  // epilogue: D[i][j] in registers, lane holds column j and rows i..i+3.
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1;
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
    for (int j = 0; j < TM; ++j) {
      const int col = tj * BM + wn * WM + j * 32 + (lane & 31);
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

template <int STAGE, bool SWAP, class TP>
__global__ __launch_bounds__(NT, 1) void ns_px_bf16(NsArgs a) {
  MMUON_RING_DECL

  const int tiles_j = a.np / PBN;
  const int tiles = (a.mp / BM) * tiles_j;
  int b, t;
  if (!decode_tile(tiles, a.N, b, t)) return;
  const int ti = t / tiles_j, tj = t % tiles_j;

  const uint16_t* P = static_cast<const uint16_t*>(a.a_in) + int64_t(b) * a.mp * a.mp +
                      int64_t(ti) * BM * a.mp;
  const uint16_t* X = static_cast<const uint16_t*>(a.x_in) + int64_t(b) * a.mp * a.np;

  f32x16 acc[TM][TM];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TM; ++j) acc[i][j] = f32x16{};
  mainloop<true, SWAP>(P, a.mp, X + tj * PBN, a.np, a.mp / BK, ring, acc);

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const float s = a.scale != nullptr ? a.scale[b] : 1.f;
  uint16_t* out = static_cast<uint16_t*>(a.out) + int64_t(b) * a.mp * a.np;
  typename TP::storage* prm = nullptr;
  if (STAGE == NS_PX_APPLY) prm = reinterpret_cast<typename TP::storage*>(a.blocks[b].param);

#pragma unroll
  for (int i = 0; i < TM; ++i) {
#pragma unroll
    for (int j = 0; j < TM; ++j) {
#pragma unroll
      for (int qg = 0; qg < 4; ++qg) {
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = acc[i][j][qg * 4 + e];
        if (SWAP) {
          // lane: row i (X' row), columns col..col+3
          const int row = ti * BM + wm * WM + i * 32 + (lane & 31);
          const int col = tj * PBN + wn * WM + j * 32 + qg * 8 + (lane >> 5) * 4;
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
          // lane: column j (X' column), rows row..row+3
          const int col = tj * PBN + wn * WM + j * 32 + (lane & 31);
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
