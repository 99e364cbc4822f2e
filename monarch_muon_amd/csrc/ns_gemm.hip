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
// (M0 holds the wave-uniform LDS base); the global address is a wave-uniform
// base plus a 32-bit per-lane byte offset.  Issued as inline assembly so that
// the compiler's wait-count pass does not guard every later LDS read with a
// vmcnt(0); the pipeline waits for exactly the slice it reads (wait_vm, in-order
// completion of vector-memory loads) and then synchronises the workgroup.
__device__ __forceinline__ void dma16(const void* base, uint32_t off, const uint16_t* lds_base) {
  const uint32_t m0 = uint32_t(reinterpret_cast<uintptr_t>((const lds_void*)lds_base));
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
               :
               : "v"(off), "s"(base), "s"(__builtin_amdgcn_readfirstlane(m0))
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

// Issue one K-major operand slice: 256 rows of 32 k at `src` (row stride ld
// elements, k offset already applied).  Wave w, instruction q covers rows
// 16*(4w+q) .. +15; lane l loads row l/4, chunk (l%4) ^ ((l>>4)&3).  `loff` is
// the lane's byte offset kmajor_lane_offset(ld).
__device__ __forceinline__ uint32_t kmajor_lane_offset(int64_t ld, int lane) {
  const int chunk = (lane & 3) ^ ((lane >> 4) & 3);
  return uint32_t((int64_t(lane >> 2) * ld + chunk * 8) * 2);
}
__device__ __forceinline__ void issue_kmajor(const uint16_t* src, int64_t ld, uint32_t loff,
                                             uint16_t* slice, int wave) {
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int grp = wave * 4 + q;
    dma16(src + int64_t(grp * 16) * ld, loff, slice + grp * 16 * BK);
  }
}

// Issue one row-major X slice: 32 rows of 256 columns at `src` (row stride ld).
// Wave w, instruction q covers rows 2*(4w+q) .. +1; lane l loads row l/32,
// physical chunk l%32 = logical granule ((l%32)/4) ^ (row & 3), chunk l%4.  The
// swizzle depends on the row's parity pair, so even and odd q use `loff[0]`,
// `loff[1]` (rowmajor_lane_offset).
__device__ __forceinline__ uint32_t rowmajor_lane_offset(int64_t ld, int lane, int qpar) {
  const int row = qpar * 2 + (lane >> 5);   // row & 3 of the instruction's rows
  const int lg = ((lane & 31) >> 2) ^ (row & 3);
  return uint32_t((int64_t(lane >> 5) * ld + lg * 32 + (lane & 3) * 8) * 2);
}
__device__ __forceinline__ void issue_rowmajor(const uint16_t* src, int64_t ld, const uint32_t (&loff)[2],
                                               uint16_t* slice, int wave) {
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int grp = wave * 4 + q;
    dma16(src + int64_t(grp * 2) * ld, loff[q & 1], slice + grp * 2 * 256);
  }
}

// 8-element K-major fragment of a 32-row MFMA operand (rows r0 + lane%32,
// k = 16*kk + 8*(lane/32) + [0,8)), r0 a multiple of 32.  The swizzle term
// ((r >> 2) & 3) only depends on lane%32, so a fragment is a per-lane base
// (kmajor_frag_base, one per kk) plus the compile-time row offset r0*BK.
__device__ __forceinline__ uint32_t kmajor_frag_base(int kk, int lane) {
  const int r = lane & 31;
  const int c = (kk * 2 + (lane >> 5)) ^ ((r >> 2) & 3);
  return uint32_t((r * BK + c * 8) * 2);
}
__device__ __forceinline__ bf16x8 frag_kmajor(const uint16_t* slice, uint32_t base, int r0) {
  return *reinterpret_cast<const bf16x8*>(reinterpret_cast<const char*>(slice) + base + r0 * BK * 2);
}

// Same fragment shape read transposed out of a row-major X slice: lane l
// receives column c0 + l%32, rows 16*kk + 8*(l/32) + [0,8).  ds_read_b64_tr_b16
// works on 16-lane groups: lane i addresses 4 elements of row i/4 at column
// 4*(i%4) of a 4x16 block and receives column i of that block.  For c0 = 32*g0
// the physical granule is g0 ^ ((l%16)/4); rowmajor_frag_base(g0) holds the
// lane's byte address for kk = 0, h = 0 and the k offsets are compile-time.
__device__ __forceinline__ uint32_t rowmajor_frag_base(int g0, int lane) {
  const int l16 = lane & 15;
  const int within = (((lane >> 4) & 1) << 4) + ((l16 & 3) << 2);
  const int k = ((lane >> 5) << 3) + (l16 >> 2);
  return uint32_t((k * 256 + ((g0 ^ (k & 3)) << 5) + within) * 2);
}
__device__ __forceinline__ bf16x8 frag_rowmajor_tr(const uint16_t* slice, uint32_t base, int kk) {
  const char* p0 = reinterpret_cast<const char*>(slice) + base + kk * 16 * 256 * 2;
  const char* p1 = p0 + 4 * 256 * 2;
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
// MFMA operand fragments of one 16-deep k step held by one wave.
struct Frags {
  bf16x8 r[TM];
  bf16x8 c[TM];
};

// Identity fragments: IDENT = 1 adds v*I on the row-operand side (acc += v X
// over the K slice that crosses the tile's diagonal rows), IDENT = 2 on the
// column-operand side (acc += v A).  v is split into two bf16 parts (hi + lo)
// so the identity term keeps ~16 bits; the products are exact and accumulate
// in fp32 with the rest of the dot product.
enum { IDENT_NONE = 0, IDENT_ROW = 1, IDENT_COL = 2 };

__device__ __forceinline__ bf16x8 ident_frag(float v, int kk, int lane) {
  // lane holds row (or column) lane%32 and k = 16*kk + 8*(lane/32) + t
  typedef short i16x8 __attribute__((ext_vector_type(8)));
  const uint16_t h = f2bf(v);
  i16x8 r = {0, 0, 0, 0, 0, 0, 0, 0};
  const int t = (lane & 31) - 16 * kk - 8 * (lane >> 5);
#pragma unroll
  for (int e = 0; e < 8; ++e) r[e] = (t == e) ? short(h) : short(0);
  return __builtin_bit_cast(bf16x8, r);
}

template <bool ROWMAJOR_C, bool SWAP, int IDENT = IDENT_NONE>
struct Pipe {
  const uint16_t* rsrc;
  int64_t rld;
  const uint16_t* csrc;
  int64_t cld;
  int KT;
  int wave, lane, wm, wn;
  uint16_t* lds;  // NSTAGE row-operand slices, then NSTAGE column-operand slices
  uint32_t r_loff, c_loff[2];     // per-lane DMA byte offsets
  uint32_t kfrag[BK / 16];        // per-lane K-major fragment bases
  uint32_t tfrag[TM];             // per-lane transposed fragment bases (one per column tile)
  int diag0;                      // K index of this wave's first identity row / column
  bf16x8 idf[BK / 16][2];         // identity fragments (hi, lo) per 16-deep k step

  __device__ __forceinline__ uint16_t* rslot(int kt) const { return lds + (kt & (NSTAGE - 1)) * SLICE; }
  __device__ __forceinline__ uint16_t* cslot(int kt) const { return lds + (NSTAGE + (kt & (NSTAGE - 1))) * SLICE; }

  __device__ __forceinline__ void issue(int kt) const {
    issue_kmajor(rsrc + kt * BK, rld, r_loff, rslot(kt), wave);
    if (ROWMAJOR_C) issue_rowmajor(csrc + int64_t(kt) * BK * cld, cld, c_loff, cslot(kt), wave);
    else issue_kmajor(csrc + kt * BK, cld, c_loff[0], cslot(kt), wave);
  }

  // Fragment reads of k step kk (0 or 1) of slice kt.
  template <int KK>
  __device__ __forceinline__ void load(int kt, Frags& f) const {
    const uint16_t* sr = rslot(kt);
    const uint16_t* sc = cslot(kt);
#pragma unroll
    for (int j = 0; j < TM; ++j)
      f.c[j] = ROWMAJOR_C ? frag_rowmajor_tr(sc, tfrag[j], KK) : frag_kmajor(sc, kfrag[KK], wn * WM + j * 32);
#pragma unroll
    for (int i = 0; i < TM; ++i) f.r[i] = frag_kmajor(sr, kfrag[KK], wm * WM + i * 32);
  }

  template <int F>
  __device__ __forceinline__ void ident_row(const Frags& f, const bf16x8 (&id)[2], f32x16 (&acc)[TM][TM]) const {
#pragma unroll
    for (int j = 0; j < TM; ++j) {
      acc[F][j] = mfma(id[0], f.c[j], acc[F][j]);
      acc[F][j] = mfma(id[1], f.c[j], acc[F][j]);
    }
  }
  template <int F>
  __device__ __forceinline__ void ident_col(const Frags& f, const bf16x8 (&id)[2], f32x16 (&acc)[TM][TM]) const {
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      acc[i][F] = mfma(f.r[i], id[0], acc[i][F]);
      acc[i][F] = mfma(f.r[i], id[1], acc[i][F]);
    }
  }

  // F >= 0: this slice crosses the identity at fragment F (32 rows/columns).
  template <int KK, int F>
  __device__ __forceinline__ void math(const Frags& f, f32x16 (&acc)[TM][TM]) const {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TM; ++j)
        acc[i][j] = SWAP ? mfma(f.c[j], f.r[i], acc[i][j]) : mfma(f.r[i], f.c[j], acc[i][j]);
    if constexpr (F >= 0) {
      if constexpr (IDENT == IDENT_ROW) ident_row<F>(f, idf[KK], acc);
      else ident_col<F>(f, idf[KK], acc);
    }
  }

  // Fragments ping-pong at half-slice granularity: the k step 1 reads of slice kt
  // stream in under the k step 0 MFMAs, and (after the slice-kt+1 barrier) the
  // k step 0 reads of slice kt+1 under the k step 1 MFMAs.  At the barrier of
  // step kt every wave has consumed slice kt-1, so its slot takes slice kt+3.
  template <int F>
  __device__ __forceinline__ void step(int kt, Frags& fa, Frags& fb, f32x16 (&acc)[TM][TM]) const {
    load<1>(kt, fb);
    math<0, F>(fa, acc);
    if (kt + 1 < KT) {
      if (kt + 2 < KT) wait_vm<2 * DMA_PER_OPERAND>();
      else wait_vm<0>();
      barrier();
      if (kt + 3 < KT) issue(kt + 3);
    }
    // unconditional so the wait counts before the second MFMA half only cover
    // fb: on the last step this reads a stale slot whose values are never used
    load<0>(kt + 1, fa);
    math<1, F>(fb, acc);
  }

  __device__ __forceinline__ void run(f32x16 (&acc)[TM][TM]) const {
    issue(0);
    if (KT > 1) issue(1);
    if (KT > 2) issue(2);
    // slice 0 visible; slices 1 and 2 may remain in flight
    if (KT > 2) wait_vm<2 * 2 * DMA_PER_OPERAND>();
    else if (KT > 1) wait_vm<2 * DMA_PER_OPERAND>();
    else wait_vm<0>();
    barrier();
    Frags fa, fb;
    load<0>(0, fa);
    if constexpr (IDENT == IDENT_NONE) {
      for (int kt = 0; kt < KT; ++kt) step<-1>(kt, fa, fb, acc);
    } else {
      // the four 32-deep slices starting at diag0 cross this wave's identity
      // fragments 0..3 in order (diag0 is a multiple of 128)
      const int kd = diag0 / BK;
      int kt = 0;
      for (; kt < kd; ++kt) step<-1>(kt, fa, fb, acc);
      step<0>(kt, fa, fb, acc);
      step<1>(kt + 1, fa, fb, acc);
      step<2>(kt + 2, fa, fb, acc);
      step<3>(kt + 3, fa, fb, acc);
      for (kt += 4; kt < KT; ++kt) step<-1>(kt, fa, fb, acc);
    }
  }
};

// ident_v: the identity scalar (IDENT_ROW / IDENT_COL); diag: K index of the
// tile's first row (IDENT_ROW) or column (IDENT_COL).
template <bool ROWMAJOR_C, bool SWAP, int IDENT = IDENT_NONE>
__device__ __forceinline__ void mainloop(const uint16_t* rsrc, int64_t rld, const uint16_t* csrc,
                                         int64_t cld, int KT, uint16_t* lds, f32x16 (&acc)[TM][TM],
                                         float ident_v = 0.f, int diag = 0) {
  Pipe<ROWMAJOR_C, SWAP, IDENT> p;
  p.rsrc = rsrc;
  p.rld = rld;
  p.csrc = csrc;
  p.cld = cld;
  p.KT = KT;
  p.lane = threadIdx.x & 63;
  p.wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  p.wm = p.wave >> 1;
  p.wn = p.wave & 1;
  p.lds = lds;
  p.r_loff = kmajor_lane_offset(rld, p.lane);
  if (ROWMAJOR_C) {
    p.c_loff[0] = rowmajor_lane_offset(cld, p.lane, 0);
    p.c_loff[1] = rowmajor_lane_offset(cld, p.lane, 1);
  } else {
    p.c_loff[0] = p.c_loff[1] = kmajor_lane_offset(cld, p.lane);
  }
#pragma unroll
  for (int kk = 0; kk < BK / 16; ++kk) p.kfrag[kk] = kmajor_frag_base(kk, p.lane);
#pragma unroll
  for (int j = 0; j < TM; ++j) p.tfrag[j] = rowmajor_frag_base(p.wn * (WM / 32) + j, p.lane);
  if constexpr (IDENT != IDENT_NONE) {
    p.diag0 = diag + (IDENT == IDENT_ROW ? p.wm : p.wn) * WM;
    const float hi = rbf(ident_v), lo = ident_v - hi;
#pragma unroll
    for (int kk = 0; kk < BK / 16; ++kk) {
      p.idf[kk][0] = ident_frag(hi, kk, p.lane);
      p.idf[kk][1] = ident_frag(lo, kk, p.lane);
    }
  }
  p.run(acc);
}

// ---------------------------------------------------------------------------
// Output staging.  After the main loop the LDS ring is idle; a 256 x 256 bf16
// tile (128 KiB) is staged there so that every global store is a coalesced
// 16-B row chunk.  Tile layout: row r is 512 B of 32 16-B chunks, chunk c of
// row r sits at c ^ (r & 31).
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t tile_off(int r, int c) {
  return uint32_t(r * 512 + ((((c >> 3) ^ (r & 31)) << 4) | ((c & 7) << 1)));
}

// Rows of the staged tile -> rows of a row-major destination (row stride ld):
// dst[r][c] = T[r][c], 16-B chunks, consecutive lanes on consecutive chunks.
__device__ __forceinline__ void tile_store_rows(const char* tile, uint16_t* dst, int64_t ld) {
  const int tid = threadIdx.x;
  const int c = (tid & 31) * 8;
#pragma unroll 4
  for (int q = 0; q < 32; ++q) {
    const int r = q * 8 + (tid >> 5);
    const uint4 v = *reinterpret_cast<const uint4*>(tile + tile_off(r, c));
    *reinterpret_cast<uint4*>(dst + int64_t(r) * ld + c) = v;
  }
}

// Columns of the staged tile -> rows of the destination: dst[i][j] = T[j][i].
// ds_read_b64_tr_b16 (16-lane groups): lane l of a group addresses T row
// j0 + l/4 at column i0 + 4*(l%4) and receives T[j0..j0+3][i0 + l]; two reads
// give 8 consecutive j of destination row i0 + l.  The four groups of a wave
// take consecutive 8-column chunks, so each destination row gets 64 contiguous
// bytes per wave.  `fn(i, j, uint4)` consumes destination row i, columns j..j+7.
template <class Fn>
__device__ __forceinline__ void tile_cols(const char* tile, Fn&& fn) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int l16 = lane & 15, grp = lane >> 4;
#pragma unroll 2
  for (int task = wave; task < 128; task += 4) {
    const int i0 = (task & 15) * 16, j0 = (task >> 4) * 32 + grp * 8;
    const int tr = j0 + (l16 >> 2), tc = i0 + ((l16 & 3) << 2);
    const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(tile + tile_off(tr, tc)));
    const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(tile + tile_off(tr + 4, tc)));
    uint4 v;
    v.x = uint32_t(uint16_t(lo[0])) | (uint32_t(uint16_t(lo[1])) << 16);
    v.y = uint32_t(uint16_t(lo[2])) | (uint32_t(uint16_t(lo[3])) << 16);
    v.z = uint32_t(uint16_t(hi[0])) | (uint32_t(uint16_t(hi[1])) << 16);
    v.w = uint32_t(uint16_t(hi[2])) | (uint32_t(uint16_t(hi[3])) << 16);
    fn(i0 + l16, j0, v);
  }
}

// Lane geometry of the D[i][j] accumulator layout of one wave: lane holds
// column j = wn*128 + 32*tj + lane%32 and rows i = wm*128 + 32*ti + 8*qg + 4*(lane/32) + e.
struct Lane {
  int lane, wm, wn;
  __device__ __forceinline__ int col(int tj) const { return wn * WM + tj * 32 + (lane & 31); }
  __device__ __forceinline__ int row(int ti, int qg) const { return wm * WM + ti * 32 + qg * 8 + (lane >> 5) * 4; }
};

// ---------------------------------------------------------------------------
// SYRK / POLY: symmetric m x m outputs, both operands K-major rows.
// ---------------------------------------------------------------------------
template <int STAGE>
__global__ __launch_bounds__(NT, 1) void ns_sym_bf16(NsArgs a) {
  __shared__ __attribute__((aligned(1024))) uint16_t lds[2 * NSTAGE * SLICE];

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
  if (STAGE == NS_SYRK)
    mainloop<false, false>(src + int64_t(ti) * BM * ld, ld, src + int64_t(tj) * BM * ld, ld, K / BK, lds, acc);
  else  // acc = A A + (b/c) A, so P = c acc = b A + c A A
    mainloop<false, false, IDENT_COL>(src + int64_t(ti) * BM * ld, ld, src + int64_t(tj) * BM * ld, ld, K / BK,
                                      lds, acc, a.cb / a.cc, tj * BM);

  // epilogue: T[j][i] = C[r0 + i][c0 + j] staged in LDS; T's rows are the mirror
  // tile C[c0 + j][r0 + i], its columns (off the diagonal) the direct tile.
  const Lane L{int(threadIdx.x & 63), int(threadIdx.x >> 6) >> 1, int(threadIdx.x >> 6) & 1};
  float f = 1.f;  // SYRK: s^2 (first iteration); POLY: c
  if (STAGE == NS_SYRK && a.scale != nullptr) {
    const float s = a.scale[b];
    f = s * s;
  }
  if (STAGE == NS_POLY) f = a.cc;
  uint16_t* out = static_cast<uint16_t*>(a.out) + int64_t(b) * a.mp * a.mp;
  const int r0 = ti * BM, c0 = tj * BM;
  char* tile = reinterpret_cast<char*>(lds);
  barrier();  // every wave is done with the ring
#pragma unroll
  for (int i = 0; i < TM; ++i) {
#pragma unroll
    for (int j = 0; j < TM; ++j) {
#pragma unroll
      for (int qg = 0; qg < 4; ++qg) {
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = f * acc[i][j][qg * 4 + e];
        *reinterpret_cast<uint2*>(tile + tile_off(L.col(j), L.row(i, qg))) =
            make_uint2(f2bf2(v[0], v[1]), f2bf2(v[2], v[3]));
      }
    }
  }
  barrier();
  tile_store_rows(tile, out + int64_t(c0) * a.mp + r0, a.mp);
  if (ti != tj) {
    uint16_t* dst = out + int64_t(r0) * a.mp + c0;
    const int64_t ldo = a.mp;
    tile_cols(tile, [&](int i, int j, const uint4& v) {
      *reinterpret_cast<uint4*>(dst + int64_t(i) * ldo + j) = v;
    });
  }
}

// ---------------------------------------------------------------------------
// PX / PX_APPLY: X' = s (a X + P X), m x n output tile (256 x 256), K = m.
// D[i][j] in registers (lane holds column j, rows i..i+3); the a X term enters
// the accumulation as (a I) X.  T[j][i] = X'[r0 + i][c0 + j] is staged in LDS;
// X' rows (PX, and the parameter rows of an untransposed block) are T's
// columns, the parameter rows of a tall block (param[j][i]) are T's rows.
// ---------------------------------------------------------------------------
constexpr int PBN = 256;                     // output tile along n

// param[o .. o+valid) += alpha * u (u = 8 bf16 in u8); one rounding to the
// parameter dtype per element, as torch's foreach add with alpha.  `vec`:
// 16-B aligned full chunk (8 bf16 = 16 B, 8 fp32 = 32 B).
template <class TP>
__device__ __forceinline__ void apply_chunk(typename TP::storage* prm, int64_t o, const uint4& u8, float alpha,
                                            int valid, bool vec) {
  const uint32_t w[4] = {u8.x, u8.y, u8.z, u8.w};
  float u[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) u[e] = __uint_as_float((e & 1) ? (w[e >> 1] & 0xffff0000u) : (w[e >> 1] << 16));
  if (vec && valid == 8) {
    if constexpr (sizeof(typename TP::storage) == 2) {
      uint4 pv = *reinterpret_cast<const uint4*>(prm + o);
      uint32_t pw[4] = {pv.x, pv.y, pv.z, pv.w};
#pragma unroll
      for (int h = 0; h < 4; ++h) {
        const float p0 = __uint_as_float(pw[h] << 16), p1 = __uint_as_float(pw[h] & 0xffff0000u);
        pw[h] = f2bf2(fmaf(alpha, u[2 * h], p0), fmaf(alpha, u[2 * h + 1], p1));
      }
      *reinterpret_cast<uint4*>(prm + o) = make_uint4(pw[0], pw[1], pw[2], pw[3]);
    } else {
      float4* q = reinterpret_cast<float4*>(prm + o);
      float4 a0 = q[0], a1 = q[1];
      a0.x = fmaf(alpha, u[0], a0.x); a0.y = fmaf(alpha, u[1], a0.y);
      a0.z = fmaf(alpha, u[2], a0.z); a0.w = fmaf(alpha, u[3], a0.w);
      a1.x = fmaf(alpha, u[4], a1.x); a1.y = fmaf(alpha, u[5], a1.y);
      a1.z = fmaf(alpha, u[6], a1.z); a1.w = fmaf(alpha, u[7], a1.w);
      q[0] = a0;
      q[1] = a1;
    }
    return;
  }
#pragma unroll
  for (int e = 0; e < 8; ++e)
    if (e < valid) TP::store(prm, o + e, fmaf(alpha, u[e], TP::load(prm, o + e)));
}

template <int STAGE, bool TRANS, class TP>
__global__ __launch_bounds__(NT, 1) void ns_px_bf16(NsArgs a) {
  __shared__ __attribute__((aligned(1024))) uint16_t lds[2 * NSTAGE * SLICE];

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
  // acc = P X + a X (the identity on the P side over the tile's diagonal rows)
  mainloop<true, false, IDENT_ROW>(P, a.mp, X + tj * PBN, a.np, a.mp / BK, lds, acc, a.ca, ti * BM);

  const Lane L{int(threadIdx.x & 63), int(threadIdx.x >> 6) >> 1, int(threadIdx.x >> 6) & 1};
  const float s = a.scale != nullptr ? a.scale[b] : 1.f;
  const int r0 = ti * BM, c0 = tj * PBN;
  char* tile = reinterpret_cast<char*>(lds);
  barrier();  // every wave is done with the ring
#pragma unroll
  for (int i = 0; i < TM; ++i) {
#pragma unroll
    for (int j = 0; j < TM; ++j) {
#pragma unroll
      for (int qg = 0; qg < 4; ++qg) {
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = s * acc[i][j][qg * 4 + e];
        *reinterpret_cast<uint2*>(tile + tile_off(L.col(j), L.row(i, qg))) =
            make_uint2(f2bf2(v[0], v[1]), f2bf2(v[2], v[3]));
      }
    }
  }
  barrier();
  if (STAGE == NS_PX) {
    uint16_t* dst = static_cast<uint16_t*>(a.out) + int64_t(b) * a.mp * a.np + int64_t(r0) * a.np + c0;
    const int64_t ldo = a.np;
    tile_cols(tile, [&](int i, int j, const uint4& v) {
      *reinterpret_cast<uint4*>(dst + int64_t(i) * ldo + j) = v;
    });
    return;
  }
  // apply: param += alpha * u; the parameter block is stored (m x n) untransposed
  // or (n x m) for a tall block
  auto* prm = reinterpret_cast<typename TP::storage*>(a.blocks[b].param);
  const float alpha = a.alpha;
  // 16-B vector access: aligned blocks and a row length that keeps chunks aligned
  const bool vec = a.vec && ((TRANS ? a.m : a.n) % 8 == 0);
  if (TRANS) {
    const int tid = threadIdx.x;
    const int c = (tid & 31) * 8;
    for (int q = 0; q < 32; ++q) {
      const int r = q * 8 + (tid >> 5);   // tile row = X' column = parameter row
      const int pr = c0 + r, pc = r0 + c;
      if (pr >= a.n || pc >= a.m) continue;
      const uint4 u8 = *reinterpret_cast<const uint4*>(tile + tile_off(r, c));
      apply_chunk<TP>(prm, int64_t(pr) * a.m + pc, u8, alpha, min(8, a.m - pc), vec);
    }
  } else {
    const int m = a.m, n = a.n;
    tile_cols(tile, [&](int i, int j, const uint4& v) {
      const int pr = r0 + i, pc = c0 + j;
      if (pr < m && pc < n) apply_chunk<TP>(prm, int64_t(pr) * n + pc, v, alpha, min(8, n - pc), vec);
    });
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
    hipLaunchKernelGGL((ns_px_bf16<STAGE, false, TP>), dim3(grid), dim3(NT), 0, s, a);
  } else {
    hipLaunchKernelGGL((ns_px_bf16<STAGE, true, TP>), dim3(grid), dim3(NT), 0, s, a);
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
