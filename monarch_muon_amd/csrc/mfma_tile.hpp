// gfx950 MFMA tile machinery shared by the Newton-Schulz and butterfly GEMMs:
// the 256 x 256 workgroup tile geometry, direct global->LDS loads, the two LDS
// slice forms and their MFMA fragment readers, and the output staging layout.
#pragma once

#include <algorithm>
#include <atomic>

#include "common.hpp"

namespace mmuon {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

constexpr int NT = 512;       // threads per workgroup (8 waves, 2 x 4)
constexpr int WG_PER_CU = 1;  // workgroups resident per CU
constexpr int BK = 32;        // K slice per pipeline stage (one panel)
constexpr int NSTAGE = 4;     // LDS ring depth: NSTAGE-2 slices in flight behind the next one
constexpr int BM = 256;       // output tile rows
constexpr int BN = 256;       // output tile columns
constexpr int WM = 128;       // wave sub-tile rows
constexpr int WN = 64;        // wave sub-tile columns
constexpr int NWN = BN / WN;  // waves along the columns
constexpr int NWAVES = NT / 64;
constexpr int TMI = WM / 32;  // 32x32 MFMA tiles per wave: 4 x 2
constexpr int TMJ = WN / 32;
constexpr int RSLICE = BM * BK;           // elements of a row-operand slice (16 KiB)
constexpr int CSLICE = BN * BK;           // elements of a column-operand slice
constexpr int SLOT = RSLICE + CSLICE;     // one ring slot
constexpr int LDS_ELEMS = NSTAGE * SLOT;
constexpr int RDMA = RSLICE * 2 / (NT * 16);  // 16-B direct loads per thread per row slice
constexpr int CDMA = CSLICE * 2 / (NT * 16);  // ... per column slice
constexpr int SLICE_DMA = RDMA + CDMA;
static_assert((BM / WM) * NWN == NWAVES, "waves tile the workgroup tile");
static_assert(LDS_ELEMS >= BN * 256, "the staged tile fits in the ring");

// Workgroups are dispatched round-robin over the 8 XCDs, and a workgroup takes
// virtual tiles w, w + G, w + 2G, ... (G = gridDim.x, a multiple of 8, every
// workgroup resident), so virtual tile w runs on XCD w % 8.  Map w to
// (block, tile) so that every tile of one block lands on the same XCD (and its
// L2), and the tiles of a block run in the same round: they start together and
// stream the block's panels in step, which the L2 serves.
__device__ __forceinline__ bool decode_tile(int w, int tiles, int N, int& b, int& t) {
  const int xcd = w & 7, local = w >> 3;
  b = xcd + 8 * (local / tiles);
  t = local % tiles;
  return b < N;
}

__device__ __forceinline__ f32x16 mfma(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// Wait until at most N vector-memory instructions of this thread are
// outstanding (they complete in issue order).
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N == 0 || N == 2 || N == 4 || N == 6 || N == 8 || N == 12, "unsupported wait count");
  if constexpr (N == 0) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  else if constexpr (N == 2) asm volatile("s_waitcnt vmcnt(2)" ::: "memory");
  else if constexpr (N == 4) asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
  else if constexpr (N == 6) asm volatile("s_waitcnt vmcnt(6)" ::: "memory");
  else if constexpr (N == 8) asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
  else asm volatile("s_waitcnt vmcnt(12)" ::: "memory");
}

// threadIdx.x through an opaque move: per-lane addresses formed from it are
// computed where they are used (once per tile) instead of being hoisted out of
// the tile loop, where they would hold registers across the main loop or be
// spilled.
__device__ __forceinline__ int fresh_tid() {
  int tid;
  asm volatile("v_mov_b32 %0, %1" : "=v"(tid) : "v"(int(threadIdx.x)));
  return tid;
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
// m0 is listed as clobbered (the asm writes it); clang warns that m0 is a
// register it reserves for its own uses, which it sets right before each.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma16(const void* base, uint32_t off, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
               :
               : "v"(off), "s"(base), "s"(__builtin_amdgcn_readfirstlane(lds))
               : "memory", "m0");
}
#pragma clang diagnostic pop

// Workgroup barrier that also stops the compiler from moving LDS reads above it.
__device__ __forceinline__ void barrier() {
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// ----- LDS layouts --------------------------------------------------------
// K-form slice [rows][32 k] (consecutive rows of one panel): a row is four
// 16-B chunks; chunk c of row r sits in slot c ^ ((r >> 2) & 3), so the 16 rows
// read by one quarter-wave's ds_read_b128 cover all 64 banks.  A direct load
// of 16 rows (1 KiB): lane l loads row l/4, chunk (l%4) ^ ((l>>4)&3)
// (kmajor_lane_offset).
// T-form slice [8 panels][32 k][32 columns]: 64-B rows as in HBM, lane l of a
// direct load takes bytes 16l..16l+15 of the 1 KiB run; the 4 rows x 64 B a
// half-wave's ds_read_b64_tr_b16 touches are 256 contiguous bytes, one access
// per bank.
__device__ __forceinline__ uint32_t kmajor_lane_offset(int lane) {
  const int chunk = (lane & 3) ^ ((lane >> 4) & 3);
  return uint32_t(((lane >> 2) * PANEL + chunk * 8) * 2);
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
// Output staging.  After the main loop the LDS ring is idle; the tile is staged
// there as T[j][i] = D[i][j] (BN rows j of 512 B) so that every global store
// is a 16-B chunk of a contiguous 1 KiB run.  Chunk c of row r sits at c ^ g(r),
// g(r) = 4 (r & 3) + ((r >> 2) & 3).  That keeps three access patterns free of
// bank conflicts: the accumulator writes (16 consecutive rows, one chunk), the
// row reads of stage_rows (4 rows x 4 chunks) and the transposed reads of
// stage_cols (4 rows x 2 chunks).
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t tile_off(int r, int c) {
  const int g = ((r & 3) << 2) | ((r >> 2) & 3);
  return uint32_t(r * 512 + ((((c >> 3) ^ g)) << 4) | ((c & 7) << 1));
}

// MFMA operand fragments of one 16-deep k step held by one wave.
struct Frags {
  bf16x8 r[TMI];
  bf16x8 c[TMJ];
};

// Persistent grid: one workgroup per CU (a multiple of 8, so that virtual tile
// v always runs on XCD v % 8), at most `total`.
inline int resident_grid(int total) {
  static std::atomic<int> cus_cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  int cus = cus_cache[dev].load(std::memory_order_relaxed);
  if (cus <= 0) {
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
      cus = 256;
    cus_cache[dev].store(cus, std::memory_order_relaxed);
  }
  return std::min(total, std::max(8, WG_PER_CU * cus / 8 * 8));
}

}  // namespace
}  // namespace mmuon
