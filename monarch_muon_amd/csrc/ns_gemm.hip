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
// mirror.  Every bf16 stack is stored in 32-column panels (panel_off), so a K
// slice is contiguous in HBM.  The X operand of PX has the contraction along its
// rows; its slice is staged into LDS as stored and read transposed with
// ds_read_b64_tr_b16.
#include <algorithm>
#include <atomic>

#include "common.hpp"
#include "kernels.hpp"

namespace mmuon {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

constexpr int NT = 256;      // threads per workgroup (4 waves, 2 x 2)
constexpr int BK = 32;       // K slice per pipeline stage (one panel)
constexpr int NSTAGE = 4;    // LDS ring depth (three slices in flight ahead of the one in use)
constexpr int BM = 256;      // output tile, both dimensions
constexpr int WM = 128;      // wave sub-tile
constexpr int TM = WM / 32;  // 32x32 MFMA tiles per wave and dimension
constexpr int SLICE = 256 * BK;          // elements of one operand slice (16 KiB)
constexpr int SLOT = 2 * SLICE;          // elements of one ring slot: row + column slice (32 KiB)
// Epilogue staging: half an output tile (128 x 256 bf16, 64 KiB) in ring slot 3
// and the 32 KiB above the ring, so ring slots 0..2 can take the next tile's
// first slices while the current tile is stored.
constexpr int STAGE_OFF = 3 * SLOT;      // elements
constexpr int LDS_ELEMS = STAGE_OFF + 128 * 256;  // 160 KiB

// Persistent workgroups: workgroup w takes virtual tiles w, w + G, w + 2G, ...
// (G = gridDim.x, a multiple of 8).  Workgroups are dispatched round-robin over
// the 8 XCDs, so virtual tile v runs on XCD v % 8; decode_tile maps v to
// (block, tile) so that every tile of one block lands on the same XCD (and its
// L2) and the tiles of a block are taken back to back.
__device__ __forceinline__ bool decode_tile(int v, int tiles, int N, int& b, int& t) {
  const int xcd = v & 7, local = v >> 3;
  b = xcd + 8 * (local / tiles);
  t = local % tiles;
  return b < N;
}

// First virtual tile >= v (stepping by the grid) whose block exists, or `total`.
__device__ __forceinline__ int next_tile(int v, int total, int tiles, int N, int& b, int& t) {
  for (; v < total; v += gridDim.x)
    if (decode_tile(v, tiles, N, b, t)) return v;
  return total;
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

// Wave-uniform scalar load of one float (SMEM path: it is not counted by vmcnt,
// so it never waits on the direct-to-LDS loads in flight).
__device__ __forceinline__ float sload_f32(const float* p) {
  float v;
  asm volatile("s_load_dword %0, %1, 0x0\n\ts_waitcnt lgkmcnt(0)" : "=s"(v) : "s"(p) : "memory");
  return v;
}

__device__ __forceinline__ f32x16 mfma(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// threadIdx.x through an opaque move: per-lane epilogue addresses derived from
// it are recomputed in every tile instead of being hoisted out of the tile loop
// (where they would stay live across the main loop and spill).
__device__ __forceinline__ int fresh_tid() {
  int t;
  asm volatile("v_mov_b32 %0, %1" : "=v"(t) : "v"(int(threadIdx.x)));
  return t;
}

// Wait until at most n vector-memory instructions of this thread are
// outstanding (they complete in issue order).  n is wave-uniform and rounded
// down to a multiple of 8 (63 at most, the counter's range), which only waits
// longer.
__device__ __forceinline__ void wait_vm(int n) {
  if (n >= 63) asm volatile("s_waitcnt vmcnt(63)" ::: "memory");
  else if (n >= 48) asm volatile("s_waitcnt vmcnt(48)" ::: "memory");
  else if (n >= 40) asm volatile("s_waitcnt vmcnt(40)" ::: "memory");
  else if (n >= 32) asm volatile("s_waitcnt vmcnt(32)" ::: "memory");
  else if (n >= 16) asm volatile("s_waitcnt vmcnt(16)" ::: "memory");
  else if (n >= 8) asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
  else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

typedef __attribute__((address_space(3))) void lds_void;

// LDS byte address of a generic pointer into LDS.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return uint32_t(reinterpret_cast<uintptr_t>((const lds_void*)p));
}

// 16-B direct global->LDS load: lane l of the wave lands at lds + 16*l (M0
// holds the wave-uniform LDS address); the global address is a wave-uniform
// base plus a 32-bit per-lane byte offset.  Issued as inline assembly so that
// the compiler's wait-count pass does not guard every later LDS read with a
// vmcnt(0); the pipeline waits for exactly the slice it reads (wait_vm, in-order
// completion of vector-memory loads) and then synchronises the workgroup.
__device__ __forceinline__ void dma16(const void* base, uint32_t off, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
               :
               : "v"(off), "s"(base), "s"(__builtin_amdgcn_readfirstlane(lds))
               : "memory");
}

// Workgroup barrier that also stops the compiler from moving LDS reads above it.
__device__ __forceinline__ void barrier() {
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// ----- LDS layouts --------------------------------------------------------
// K-major slice [256 rows][32 k] (256 rows of one panel): a row is four 16-B
// chunks; chunk c of row r sits in slot c ^ ((r >> 2) & 3), so the 16 rows read
// by one quarter-wave's ds_read_b128 cover all 64 banks.
// X slice of a PX stage [8 panels][32 k][32 columns]: 64-B rows as in HBM; the
// 4 rows x 64 B a half-wave's ds_read_b64_tr_b16 touches are 256 contiguous
// bytes, one access per bank.

// Issue one K-major operand slice: 256 consecutive panel rows at `src`, one
// contiguous 16 KiB run.  Wave w, instruction q covers rows 16*(4w+q) .. +15
// (1 KiB); lane l loads row l/4, chunk (l%4) ^ ((l>>4)&3) (kmajor_lane_offset).
__device__ __forceinline__ uint32_t kmajor_lane_offset(int lane) {
  const int chunk = (lane & 3) ^ ((lane >> 4) & 3);
  return uint32_t(((lane >> 2) * PANEL + chunk * 8) * 2);
}
__device__ __forceinline__ void issue_kmajor(const uint16_t* src, uint32_t loff, uint32_t slice, int wave) {
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int grp = wave * 4 + q;
    dma16(src + grp * 16 * PANEL, loff, slice + grp * 1024);
  }
}

// Issue one X slice of a PX stage: rows k0 .. k0+31 of the 8 column panels at
// src, src + pstride, ... (2 KiB contiguous each).  Wave w, instruction q covers
// panel (4w+q)/2, rows 16*((4w+q)%2) .. +15; the lane offset is 16*l bytes.
__device__ __forceinline__ void issue_xslice(const uint16_t* src, int64_t pstride, uint32_t loff,
                                             uint32_t slice, int wave) {
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int grp = wave * 4 + q;
    dma16(src + (grp >> 1) * pstride + (grp & 1) * 16 * PANEL, loff, slice + grp * 1024);
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

// Same fragment shape read transposed out of an X slice: lane l receives
// column 32*jb + l%32, rows 16*kk + 8*(l/32) + [0,8).  ds_read_b64_tr_b16 works
// on 16-lane groups: lane i addresses 4 elements of row i/4 at column 4*(i%4)
// of a 4x16 block and receives column i of that block; lanes 16..31 take the
// panel's columns 16..31.  rowmajor_frag_base(jb) is the lane's byte address
// for kk = 0 and the first four rows; the k offsets are compile-time.
__device__ __forceinline__ uint32_t rowmajor_frag_base(int jb, int lane) {
  const int l16 = lane & 15;
  const int col = (((lane >> 4) & 1) << 4) + ((l16 & 3) << 2);
  const int k = ((lane >> 5) << 3) + (l16 >> 2);
  return uint32_t(jb * 2048 + k * 64 + col * 2);
}
__device__ __forceinline__ bf16x8 frag_rowmajor_tr(const uint16_t* slice, uint32_t base, int kk) {
  const char* p0 = reinterpret_cast<const char*>(slice) + base + kk * 16 * 64;
  const char* p1 = p0 + 4 * 64;
  const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p0));
  const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p1));
  typedef short i16x8 __attribute__((ext_vector_type(8)));
  const i16x8 v = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  return __builtin_bit_cast(bf16x8, v);
}

// ---------------------------------------------------------------------------
// The pipelined main loop shared by every stage.  ROWMAJOR_C: the column
// operand is the X stack read transposed (PX stages), else K-major (SYRK/POLY).
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

template <bool ROWMAJOR_C, int IDENT = IDENT_NONE>
struct Pipe {
  // per tile
  const uint16_t* rsrc;  // row operand: panel 0, first row of the tile
  const uint16_t* csrc;  // column operand: panel 0, first row (K-major) / first panel (X)
  int diag0;             // K index of this wave's first identity row / column
  // per launch
  int64_t pstride;       // elements per panel of the row operand (rows * 32)
  int64_t cstride;       // elements per panel of the column operand
  int KT;
  int wave, lane, wm, wn;
  uint16_t* lds;  // ring slot s at lds + s*SLOT: row-operand slice, then column-operand slice
  uint32_t lds0;  // LDS byte address of lds
  uint32_t r_loff, c_loff;        // per-lane DMA byte offsets
  uint32_t kfrag[BK / 16];        // per-lane K-major fragment bases
  uint32_t tfrag[TM];             // per-lane transposed fragment bases (one per column tile)
  float id_hi, id_lo;             // identity scalar split into two bf16 parts

  __device__ __forceinline__ void init(int64_t pstride_, int64_t cstride_, int KT_, uint16_t* lds_,
                                       float ident_v) {
    pstride = pstride_;
    cstride = cstride_;
    KT = KT_;
    lane = threadIdx.x & 63;
    wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    wm = wave >> 1;
    wn = wave & 1;
    lds = lds_;
    lds0 = lds_addr(lds_);
    r_loff = kmajor_lane_offset(lane);
    c_loff = ROWMAJOR_C ? uint32_t(lane * 16) : r_loff;
#pragma unroll
    for (int kk = 0; kk < BK / 16; ++kk) kfrag[kk] = kmajor_frag_base(kk, lane);
#pragma unroll
    for (int j = 0; j < TM; ++j) tfrag[j] = rowmajor_frag_base(wn * (WM / 32) + j, lane);
    id_hi = rbf(ident_v);
    id_lo = ident_v - id_hi;
  }

  // rsrc_ / csrc_: panel-layout operands at the tile's first row (first panel
  // for the X operand of PX); diag: K index of the tile's first row (IDENT_ROW)
  // or column (IDENT_COL).
  __device__ __forceinline__ void set_tile(const uint16_t* rsrc_, const uint16_t* csrc_, int diag) {
    rsrc = rsrc_;
    csrc = csrc_;
    diag0 = diag + (IDENT == IDENT_ROW ? wm : wn) * WM;
  }

  __device__ __forceinline__ uint16_t* rslot(int kt) const { return lds + (kt & (NSTAGE - 1)) * SLOT; }
  __device__ __forceinline__ uint16_t* cslot(int kt) const { return rslot(kt) + SLICE; }

  __device__ __forceinline__ void issue(int kt) const {
    const uint32_t rs = lds0 + (kt & (NSTAGE - 1)) * SLOT * 2;
    const uint32_t cs = rs + SLICE * 2;
    issue_kmajor(rsrc + kt * pstride, r_loff, rs, wave);
    if (ROWMAJOR_C) issue_xslice(csrc + kt * BK * PANEL, cstride, c_loff, cs, wave);
    else issue_kmajor(csrc + kt * cstride, r_loff, cs, wave);
  }

  // Slices 0..2 of the tile into ring slots 0..2 (slot 3 stays free for the
  // epilogue staging).  Slice 0 is issued before the previous tile's epilogue
  // stores, slices 1 and 2 after them, so only the wait for slice 0 has to
  // allow for the stores.
  __device__ __forceinline__ void prologue_first() const { issue(0); }
  __device__ __forceinline__ void prologue_rest() const {
    if (KT > 1) issue(1);
    if (KT > 2) issue(2);
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

  // F >= 0: this slice crosses the identity at fragment F (32 rows/columns);
  // the identity fragments of k step KK are built on the spot.
  template <int KK, int F>
  __device__ __forceinline__ void math(const Frags& f, f32x16 (&acc)[TM][TM]) const {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TM; ++j) acc[i][j] = mfma(f.r[i], f.c[j], acc[i][j]);
    if constexpr (F >= 0) {
      const bf16x8 ih = ident_frag(id_hi, KK, lane), il = ident_frag(id_lo, KK, lane);
      if constexpr (IDENT == IDENT_ROW) {
#pragma unroll
        for (int j = 0; j < TM; ++j) {
          acc[F][j] = mfma(ih, f.c[j], acc[F][j]);
          acc[F][j] = mfma(il, f.c[j], acc[F][j]);
        }
      } else {
#pragma unroll
        for (int i = 0; i < TM; ++i) {
          acc[i][F] = mfma(f.r[i], ih, acc[i][F]);
          acc[i][F] = mfma(f.r[i], il, acc[i][F]);
        }
      }
    }
  }

  // Fragments ping-pong at half-slice granularity: the k step 1 reads of slice kt
  // stream in under the k step 0 MFMAs, and (after the slice-kt+1 barrier) the
  // k step 0 reads of slice kt+1 under the k step 1 MFMAs.  At the barrier of
  // step kt every wave has consumed slice kt-1, so its slot takes slice kt+3.
  // Step kt waits for slice kt+1, with slice kt+2 allowed in flight.
  template <int F>
  __device__ __forceinline__ void step(int kt, Frags& fa, Frags& fb, f32x16 (&acc)[TM][TM]) const {
    load<1>(kt, fb);
    math<0, F>(fa, acc);
    if (kt + 1 < KT) {
      if (kt + 2 < KT) wait_vm(8);
      else wait_vm(0);
      barrier();
      if (kt + 3 < KT) issue(kt + 3);
    }
    // unconditional so the wait counts before the second MFMA half only cover
    // fb: on the last step this reads a stale slot whose values are never used
    load<0>(kt + 1, fa);
    math<1, F>(fb, acc);
  }

  // The tile's main loop, after prologue_first() and prologue_rest().  extra:
  // vector-memory instructions this thread issued between the two (the previous
  // tile's epilogue stores); they complete in order behind slice 0.
  __device__ __forceinline__ void run(f32x16 (&acc)[TM][TM], int extra) const {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TM; ++j) acc[i][j] = f32x16{};
    // slice 0 visible; the stores and slices 1 and 2 may remain in flight
    wait_vm(8 * (KT > 2 ? 2 : KT - 1) + extra);
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

// ---------------------------------------------------------------------------
// Output staging.  T[j][i] = D[i][j] (the accumulator tile, lane-major in j) is
// staged in LDS half at a time (T rows 128h .. 128h+127, 64 KiB) so that every
// global store is a 16-B chunk of a contiguous 1 KiB run.  Staged row r is 512 B
// of 32 16-B chunks; chunk c sits at c ^ g(r), g(r) = 4 (r & 3) + ((r >> 2) & 3).
// That keeps three access patterns free of bank conflicts: the accumulator
// writes (16 consecutive rows, one chunk), the row reads of stage_rows (4 rows x
// 4 chunks) and the transposed reads of stage_cols (4 rows x 2 chunks).
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t tile_off(int r, int c) {
  const int g = ((r & 3) << 2) | ((r >> 2) & 3);
  return uint32_t(r * 512 + ((((c >> 3) ^ g)) << 4) | ((c & 7) << 1));
}

// Lane geometry of the D[i][j] accumulator layout of one wave: lane holds
// column j = wn*128 + 32*tj + lane%32 and rows i = wm*128 + 32*ti + 8*qg + 4*(lane/32) + e.
struct Lane {
  int lane, wm, wn;
  __device__ __forceinline__ int col(int tj) const { return wn * WM + tj * 32 + (lane & 31); }
  __device__ __forceinline__ int row(int ti, int qg) const { return wm * WM + ti * 32 + qg * 8 + (lane >> 5) * 4; }
};

// Half h of T (rows j = 128h + r) into the staging area: the two waves with
// wn == h own those columns of D.  f scales every value before the bf16 rounding.
__device__ __forceinline__ void stage_half(char* stage, const f32x16 (&acc)[TM][TM], const Lane& L, float f) {
#pragma unroll
  for (int i = 0; i < TM; ++i) {
#pragma unroll
    for (int j = 0; j < TM; ++j) {
#pragma unroll
      for (int qg = 0; qg < 4; ++qg) {
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = f * acc[i][j][qg * 4 + e];
        *reinterpret_cast<uint2*>(stage + tile_off(j * 32 + (L.lane & 31), L.row(i, qg))) =
            make_uint2(f2bf2(v[0], v[1]), f2bf2(v[2], v[3]));
      }
      // one 32x32 block at a time: keeps the accumulator reads from being
      // hoisted (and their values held in VGPRs) across the whole tile
      __builtin_amdgcn_sched_barrier(0);
    }
  }
}

// Staged rows -> a panel-layout destination with the same rows: dst[r][i] =
// S[r][i] for the 128 staged rows, dst at the first staged row of the tile's
// first column panel.  One wave instruction writes rows 16u .. 16u+15 of one
// panel (1 KiB contiguous); 16 stores per thread.
__device__ __forceinline__ void stage_rows(const char* stage, uint16_t* dst, int64_t pstride, int tid) {
  const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
#pragma unroll 4
  for (int it = 0; it < 16; ++it) {
    const int u = wave + 4 * it;  // 8 panels x 8 row blocks
    const int q = u & 7, r = (u >> 3) * 16 + (lane >> 2);
    const int i = q * 32 + (lane & 3) * 8;
    const uint4 v = *reinterpret_cast<const uint4*>(stage + tile_off(r, i));
    *reinterpret_cast<uint4*>(dst + q * pstride + r * PANEL + (lane & 3) * 8) = v;
  }
}

// Staged columns -> rows of the destination: dst[i][r] = S[r][i] (256 rows i,
// 128 columns r).  ds_read_b64_tr_b16 (16-lane groups): lane l of a group
// addresses S row r0 + l/4 at column i0 + 4*(l%4) and receives S[r0..r0+3][i0 + l];
// two reads give 8 consecutive r of destination row i0 + l.  The four groups of
// a wave take consecutive 8-column chunks, so one wave instruction covers
// destination rows i0 .. i0+15, columns 32t .. 32t+31: one panel's contiguous
// 1 KiB.  `fn(i, r, uint4)` consumes destination row i, columns r..r+7; 16
// calls per thread.
template <class Fn>
__device__ __forceinline__ void stage_cols(const char* stage, int tid, Fn&& fn) {
  const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15, grp = lane >> 4;
#pragma unroll 2
  for (int task = wave; task < 64; task += 4) {
    const int i0 = (task & 15) * 16, r0 = (task >> 4) * 32 + grp * 8;
    const int tr = r0 + (l16 >> 2), tc = i0 + ((l16 & 3) << 2);
    const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(stage + tile_off(tr, tc)));
    const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(stage + tile_off(tr + 4, tc)));
    uint4 v;
    v.x = uint32_t(uint16_t(lo[0])) | (uint32_t(uint16_t(lo[1])) << 16);
    v.y = uint32_t(uint16_t(lo[2])) | (uint32_t(uint16_t(lo[3])) << 16);
    v.z = uint32_t(uint16_t(hi[0])) | (uint32_t(uint16_t(hi[1])) << 16);
    v.w = uint32_t(uint16_t(hi[2])) | (uint32_t(uint16_t(hi[3])) << 16);
    fn(i0 + l16, r0, v);
  }
}

// ---------------------------------------------------------------------------
// SYRK / POLY: symmetric m x m outputs, both operands K-major rows.  Persistent:
// after a tile's main loop the next tile's first three slices are issued before
// the tile is stored, so their latency and the stores overlap.
// ---------------------------------------------------------------------------
template <int STAGE>
__global__ __launch_bounds__(NT, 1) void ns_sym_bf16(NsArgs a) {
  __shared__ __attribute__((aligned(1024))) uint16_t lds[LDS_ELEMS];
  char* stage = reinterpret_cast<char*>(lds + STAGE_OFF);

  const int nt = a.mp / BM;
  const int tiles = nt * (nt + 1) / 2;
  const int total = 8 * ((a.N + 7) / 8) * tiles;
  const int K = STAGE == NS_SYRK ? a.kx : a.mp;
  const int64_t pstride = int64_t(a.mp) * PANEL;
  const uint16_t* base = static_cast<const uint16_t*>(STAGE == NS_SYRK ? a.x_in : a.a_in);
  const int64_t bstride = int64_t(a.mp) * (STAGE == NS_SYRK ? a.np : a.mp);
  const int wn = (threadIdx.x >> 6) & 1;

  // POLY: acc = A A + (b/c) A, so P = c acc = b A + c A A
  Pipe<false, STAGE == NS_POLY ? IDENT_COL : IDENT_NONE> p;
  p.init(pstride, pstride, K / BK, lds, STAGE == NS_POLY ? a.cb / a.cc : 0.f);

  int b, t;
  int v = next_tile(blockIdx.x, total, tiles, a.N, b, t);
  if (v >= total) return;
  int ti, tj;
  sym_tile(t, nt, ti, tj);
  p.set_tile(base + b * bstride + ti * BM * PANEL, base + b * bstride + tj * BM * PANEL, tj * BM);
  p.prologue_first();
  p.prologue_rest();
  int extra = 0;
  f32x16 acc[TM][TM];
  while (true) {
    p.run(acc, extra);
    barrier();  // every wave is done with the ring
    const int cb = b, cti = ti, ctj = tj;
    v = next_tile(v + gridDim.x, total, tiles, a.N, b, t);
    if (v < total) {
      sym_tile(t, nt, ti, tj);
      p.set_tile(base + b * bstride + ti * BM * PANEL, base + b * bstride + tj * BM * PANEL, tj * BM);
      p.prologue_first();
    }
    // epilogue: T[j][i] = C[r0 + i][c0 + j]; T's rows are the mirror tile
    // C[c0 + j][r0 + i] (the only write on the diagonal), its columns the direct tile.
    const int tid = fresh_tid();
    const Lane L{tid & 63, (tid >> 6) >> 1, (tid >> 6) & 1};
    float f = STAGE == NS_POLY ? a.cc : 1.f;  // SYRK: s^2 on the first iteration
    if (STAGE == NS_SYRK && a.scale != nullptr) {
      const float sc = sload_f32(a.scale + cb);
      f = sc * sc;
    }
    uint16_t* out = static_cast<uint16_t*>(a.out) + cb * int64_t(a.mp) * a.mp;
    const int r0 = cti * BM, c0 = ctj * BM;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      if (wn == h) stage_half(stage, acc, L, f);
      barrier();
      stage_rows(stage, out + (r0 / PANEL) * pstride + int64_t(c0 + 128 * h) * PANEL, pstride, tid);
      if (cti != ctj) {
        uint16_t* dst = out + ((c0 + 128 * h) / PANEL) * pstride + int64_t(r0) * PANEL;
        stage_cols(stage, tid, [&](int i, int r, const uint4& u) {
          *reinterpret_cast<uint4*>(dst + (r >> 5) * pstride + i * PANEL + (r & 31)) = u;
        });
      }
      if (h == 0) barrier();  // half 1 overwrites the staging area
    }
    if (v >= total) break;
    p.prologue_rest();
    extra = cti != ctj ? 64 : 32;  // stores per thread issued after slice 0
  }
}

// ---------------------------------------------------------------------------
// PX / PX_APPLY: X' = s (a X + P X), m x n output tile (256 x 256), K = m.
// D[i][j] in registers (lane holds column j, rows i..i+3); the a X term enters
// the accumulation as (a I) X.  T[j][i] = X'[r0 + i][c0 + j] is staged in LDS;
// X' rows (PX, and the parameter rows of an untransposed block) are T's
// columns, the parameter rows of a tall block (param[j][i]) are T's rows.
// PX is persistent like ns_sym_bf16; PX_APPLY issues the next tile's slices
// after its parameter updates (which load the parameters).
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
  __shared__ __attribute__((aligned(1024))) uint16_t lds[LDS_ELEMS];
  char* stage = reinterpret_cast<char*>(lds + STAGE_OFF);
  constexpr bool APPLY = STAGE == NS_PX_APPLY;

  const int tiles_j = a.np / PBN;
  const int tiles = (a.mp / BM) * tiles_j;
  const int total = 8 * ((a.N + 7) / 8) * tiles;
  const int64_t pstride = int64_t(a.mp) * PANEL;
  const uint16_t* Pbase = static_cast<const uint16_t*>(a.a_in);
  const uint16_t* Xbase = static_cast<const uint16_t*>(a.x_in);
  const int wn = (threadIdx.x >> 6) & 1;

  // acc = P X + a X (the identity on the P side over the tile's diagonal rows)
  Pipe<true, IDENT_ROW> p;
  p.init(pstride, pstride, a.mp / BK, lds, a.ca);
  auto set = [&](int b, int t) {
    const int ti = t / tiles_j, tj = t % tiles_j;
    p.set_tile(Pbase + b * int64_t(a.mp) * a.mp + ti * BM * PANEL,
               Xbase + b * int64_t(a.mp) * a.np + (tj * PBN / PANEL) * pstride, ti * BM);
  };

  int b, t;
  int v = next_tile(blockIdx.x, total, tiles, a.N, b, t);
  if (v >= total) return;
  set(b, t);
  p.prologue_first();
  p.prologue_rest();
  int extra = 0;
  f32x16 acc[TM][TM];
  while (true) {
    p.run(acc, extra);
    barrier();  // every wave is done with the ring
    const int cb = b, cti = t / tiles_j, ctj = t % tiles_j;
    v = next_tile(v + gridDim.x, total, tiles, a.N, b, t);
    if (!APPLY && v < total) {
      set(b, t);
      p.prologue_first();
    }
    const float s = a.scale != nullptr ? sload_f32(a.scale + cb) : 1.f;
    const int r0 = cti * BM, c0 = ctj * PBN;
    const int tid = fresh_tid();
    const Lane L{tid & 63, (tid >> 6) >> 1, (tid >> 6) & 1};
    if constexpr (!APPLY) {
      uint16_t* out = static_cast<uint16_t*>(a.out) + cb * int64_t(a.mp) * a.np;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        if (wn == h) stage_half(stage, acc, L, s);
        barrier();
        // X'[r0 + i][c0 + 128h + r] = S[r][i]
        uint16_t* dst = out + ((c0 + 128 * h) / PANEL) * pstride + int64_t(r0) * PANEL;
        stage_cols(stage, tid, [&](int i, int r, const uint4& u) {
          *reinterpret_cast<uint4*>(dst + (r >> 5) * pstride + i * PANEL + (r & 31)) = u;
        });
        if (h == 0) barrier();
      }
      if (v < total) p.prologue_rest();
      extra = 32;  // stores per thread issued after slice 0
    } else {
      // apply: param += alpha * u; the parameter block is stored (m x n)
      // untransposed or (n x m) for a tall block
      auto* prm = reinterpret_cast<typename TP::storage*>(a.blocks[cb].param);
      const float alpha = a.alpha;
      const int m = a.m, n = a.n;
      // 16-B vector access: aligned blocks and a row length that keeps chunks aligned
      const bool vec = a.vec && ((TRANS ? m : n) % 8 == 0);
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        if (wn == h) stage_half(stage, acc, L, s);
        barrier();
        const int cj = c0 + 128 * h;  // first X' column of this half
        if (TRANS) {
          const int c = (tid & 31) * 8;
          for (int q = 0; q < 16; ++q) {
            const int r = q * 8 + (tid >> 5);  // staged row = X' column = parameter row
            const int pr = cj + r, pc = r0 + c;
            if (pr >= n || pc >= m) continue;
            const uint4 u8 = *reinterpret_cast<const uint4*>(stage + tile_off(r, c));
            apply_chunk<TP>(prm, int64_t(pr) * m + pc, u8, alpha, min(8, m - pc), vec);
          }
        } else {
          stage_cols(stage, tid, [&](int i, int r, const uint4& u) {
            const int pr = r0 + i, pc = cj + r;
            if (pr < m && pc < n) apply_chunk<TP>(prm, int64_t(pr) * n + pc, u, alpha, min(8, n - pc), vec);
          });
        }
        barrier();  // the staging area is reused (next half, or the next tile's slot 3)
      }
      if (v < total) {
        set(b, t);
        p.prologue_first();
        p.prologue_rest();
      }
      extra = 0;
    }
    if (v >= total) break;
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

// Persistent grid: one workgroup per CU (each takes all of a CU's LDS), a
// multiple of 8 so that a workgroup's tiles stay on its XCD.
int persistent_grid(int total) {
  static std::atomic<int> cus_cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  int cus = cus_cache[dev].load(std::memory_order_relaxed);
  if (cus <= 0) {
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
      cus = 256;
    cus_cache[dev].store(cus, std::memory_order_relaxed);
  }
  const int g = std::max(8, cus / 8 * 8);
  return std::min(total, g);
}

template <int STAGE, class TP>
void launch_bf16(const NsArgs& a, hipStream_t s) {
  const int nb8 = 8 * ((a.N + 7) / 8);
  if constexpr (STAGE == NS_SYRK || STAGE == NS_POLY) {
    const int nt = a.mp / BM;
    const dim3 grid(persistent_grid(nb8 * (nt * (nt + 1) / 2)));
    hipLaunchKernelGGL((ns_sym_bf16<STAGE>), grid, dim3(NT), 0, s, a);
  } else {
    const dim3 grid(persistent_grid(nb8 * (a.mp / BM) * (a.np / PBN)));
    if constexpr (STAGE == NS_PX) {
      hipLaunchKernelGGL((ns_px_bf16<STAGE, false, TP>), grid, dim3(NT), 0, s, a);
    } else {
      if (!a.transposed) hipLaunchKernelGGL((ns_px_bf16<STAGE, false, TP>), grid, dim3(NT), 0, s, a);
      else hipLaunchKernelGGL((ns_px_bf16<STAGE, true, TP>), grid, dim3(NT), 0, s, a);
    }
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
