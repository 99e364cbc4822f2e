// Newton-Schulz quintic as a chain of batched gfx950 MFMA GEMM stages.
//
// One Newton-Schulz iteration over a stack of N blocks X (m x n, m <= n):
//   SYRK : A = s^2 * X X^T                      (m x m, symmetric, K = n)
//   POLY : P = a I + b A + c A A                (m x m, symmetric, K = m)
//   PX   : X' = s * P X                         (m x n, K = m)
//   PX_APPLY (last iteration): param += alpha * bf16(X') written straight into
//          the parameter blocks, un-transposed for tall blocks.
//   SYMM : C = S1 S2 of two symmetric stacks that commute (the Gram form of the
//          rectangular groups: iterations on m x m polynomials of X0 X0^T; the
//          launch plans are built in abi.hip)
// s = 1/(||X0||_F + 1e-7) on the first iteration (the Frobenius normalisation
// folded into the products: (sX)(sX)^T = s^2 XX^T and P(sX) = s PX), 1
// afterwards.  The a X term of the quintic is carried by P's diagonal: POLY adds
// a to its fp32 diagonal before the one bf16 rounding of P (the reference rounds
// a X to bf16 in the same way), so PX is a plain product.
//
// bf16 kernels: v_mfma_f32_32x32x16_bf16, fp32 accumulation, bf16 stage outputs.
// One 512-thread workgroup (8 waves, 2 per SIMD) per CU computes 256 x 256
// output tiles, each wave a 128 x 64 sub-tile (4 x 2 MFMA tiles, 128
// accumulators).  K advances 32 at a time through a 4-slot LDS ring filled by
// direct global->LDS loads (global_load_lds_dwordx4), two slices in flight
// behind the one being read; the loads of a step are interleaved with its
// MFMAs.  The workgroups are persistent and walk the tiles in rounds, all tiles
// of one block on one XCD.  Every bf16 stack is stored in 32-column panels
// (panel_off), so a K slice is one contiguous run in HBM.  The symmetric A and
// P stacks hold only their tiles on and above the diagonal: SYRK and POLY
// compute and store just those, and their consumers read the missing part as
// the transpose of the stored part (ds_read_b64_tr_b16), as PX reads X.
#include <algorithm>
#include <atomic>

#include "common.hpp"
#include "kernels.hpp"
#include "mfma_tile.hpp"

namespace mmuon {
namespace {

// Tiles of a symmetric m x m product: BM-row band ti, BN-column band tc with
// tc >= R ti, R = BM / BN (the upper triangle and the diagonal blocks), ti-major.
constexpr int R_SYM = BM / BN;
__device__ __forceinline__ void sym_tile(int t, int nc, int& ti, int& tc) {
  int i = 0;
  while (t >= nc - R_SYM * i) {
    t -= nc - R_SYM * i;
    ++i;
  }
  ti = i;
  tc = R_SYM * i + t;
}

// ---------------------------------------------------------------------------
// The pipelined main loop shared by every stage.  Each operand slice (256
// operand rows x 32 k) is read in one of two forms:
//   K: K-major, rows of the operand itself (one contiguous 16 KiB run of a panel);
//   T: transposed, 32 rows of the 8 panels whose columns are the operand's rows
//      (2 KiB runs), read with ds_read_b64_tr_b16.
// The X operand of PX is always T.  Gram and polynomial stacks store only the
// tiles on and above the diagonal, so an operand band R of them is T for the
// K slices left of its diagonal block (from the stored tile (kb, R)) and K from
// there on.  A slice pair (row operand, column operand) is KK, KT or TT.
// ---------------------------------------------------------------------------
// Identity term folded into the accumulation: IDENT_COL adds v A (A: the row
// operand) over the K slices that cross the tile's diagonal columns.  The
// values are taken from the slice in LDS and enter the fp32 accumulators by
// FMA (Pipe::ident_add).
enum { IDENT_NONE = 0, IDENT_COL = 2 };

enum { OP_K = 0, OP_T = 1, OP_SPLIT = 2 };  // operand form over K: always K, always T, T then K
enum { M_KK = 0, M_KT = 1, M_TT = 2 };        // forms of one slice pair (row, column)
constexpr bool row_t(int m) { return m == M_TT; }
constexpr bool col_t(int m) { return m != M_KK; }

// MASK: the wave's 32x32 MFMA tiles (bit i*TMJ + j) that are computed; the
// others, and the fragment reads only they need, are left out.
// SHARED: the row and column operands are the same rows (a diagonal tile of a
// symmetric product): only the row-operand slice is loaded, and the column
// fragments are read from it.
template <int RK, int CK, int IDENT, int MASK = 0xFF, bool SHARED = false>
struct Pipe {
  static_assert(RDMA == 2 && CDMA == 2, "two direct loads per thread and operand slice");
  static constexpr int DMA = SHARED ? RDMA : SLICE_DMA;  // direct loads per thread and slice
  static constexpr bool tile_on(int i, int j) { return (MASK >> (i * TMJ + j)) & 1; }
  // fragment read G (column fragments first, then row fragments) feeds a computed tile
  static constexpr bool frag_on(int G) {
    bool on = false;
    if (G < TMJ) {
      for (int i = 0; i < TMI; ++i) on = on || tile_on(i, G);
    } else {
      for (int j = 0; j < TMJ; ++j) on = on || tile_on(G - TMJ, j);
    }
    return on;
  }
  static_assert(RK != OP_T && (RK == OP_K || CK != OP_K), "row T only where the column is T");
  // the last run of slices: column T throughout (PX), else both K
  static constexpr int ML = CK == OP_T ? M_KT : M_KK;
  const uint16_t* rsrc_k;  // row operand K form: panel 0 at the operand's first row
  const uint16_t* rsrc_t;  // row operand T form: row 0 of the first panel holding its rows
  const uint16_t* csrc_k;
  const uint16_t* csrc_t;
  int thr_r, thr_c;        // OP_SPLIT: slices kt < thr are T
  uint32_t pstride_b;      // bytes per panel (rows * 32 * 2; a block is below 2^31 bytes)
  int KT;
  int wave, lane, wm, wn;
  uint16_t* lds;  // ring slot s at lds + s*SLOT: row-operand slice, then column-operand slice
  uint32_t lds0;  // LDS byte address of lds
  uint32_t k_loff;                // per-lane direct-load byte offset of the K form (T form: 16 * lane)
  uint32_t kfrag[BK / 16];        // per-lane K-form fragment bases
  uint32_t tfrag_r, tfrag_c;      // per-lane T-form fragment bases of the wave's first row / column tile
  int diag0;                      // K index of this wave's first identity column
  float id_v;                     // identity scalar

  __device__ __forceinline__ uint16_t* rslot(int kt) const { return lds + (uint32_t(kt) % NSTAGE) * SLOT; }

  __device__ __forceinline__ bool row_is_t(int kt) const { return RK == OP_SPLIT && kt < thr_r; }
  __device__ __forceinline__ bool col_is_t(int kt) const {
    return CK == OP_T || (CK == OP_SPLIT && kt < thr_c);
  }

  // Direct load Q (0, 1: row operand; 2, 3: column operand) of slice src_kt into
  // the ring slot of slice slot_kt (the same slice, except for the harmless
  // refill of a consumed slot at the end of the loop).  K form: wave w, load q
  // covers operand rows 16 (2w + q) .. +15 of the panel (1 KiB); T form: panel
  // w of the operand, k rows 16q .. 16q+15 of the slice (1 KiB).  Either way the
  // load lands at byte (2w + q) * 1024 of the operand's slice.
  // RF >= 0: the slice pair is in form RF (known when the slice lies in the same
  // run as the step that loads it); RF < 0: decided from the slice index.
  template <int Q, int RF = -1>
  __device__ __forceinline__ void issue_one(int src_kt, int slot_kt) const {
    constexpr int q = Q & 1;
    const uint32_t dst =
        lds0 + (uint32_t(slot_kt) % NSTAGE) * SLOT * 2 + (Q < 2 ? 0 : RSLICE * 2) + (2 * wave + q) * 1024;
    bool t;
    if constexpr (RF >= 0) t = Q < 2 ? row_t(RF) : col_t(RF);
    else t = Q < 2 ? row_is_t(src_kt) : col_is_t(src_kt);
    const uint16_t* srck = Q < 2 ? rsrc_k : csrc_k;
    const uint16_t* srct = Q < 2 ? rsrc_t : csrc_t;
    // 32-bit byte offsets from the operand's base
    const uint32_t ks = uint32_t(src_kt);
    if (t)
      dma16(reinterpret_cast<const char*>(srct) + (ks * (BK * PANEL * 2) + uint32_t(wave) * pstride_b + q * 16 * PANEL * 2),
            uint32_t(lane) << 4, dst);
    else
      dma16(reinterpret_cast<const char*>(srck) + (ks * pstride_b + uint32_t(2 * wave + q) * (16 * PANEL * 2)), k_loff,
            dst);
  }
  __device__ __forceinline__ void issue(int src_kt, int slot_kt) const {
    issue_one<0>(src_kt, slot_kt);
    issue_one<1>(src_kt, slot_kt);
    if constexpr (!SHARED) {
      issue_one<2>(src_kt, slot_kt);
      issue_one<3>(src_kt, slot_kt);
    }
  }

  // Fragment read G (column fragments first, then row fragments) of k step KK
  // of slice kt in slice-pair form M.
  template <int KK, int G, int M>
  __device__ __forceinline__ void load_one(int kt, Frags& f) const {
    const uint16_t* sr = rslot(kt);
    const uint16_t* sc = SHARED ? sr : sr + RSLICE;
    if constexpr (G < TMJ)
      f.c[G] = col_t(M) ? frag_rowmajor_tr(sc, tfrag_c + G * 2048, KK) : frag_kmajor(sc, kfrag[KK], wn * WN + G * 32);
    else
      f.r[G - TMJ] = row_t(M) ? frag_rowmajor_tr(sr, tfrag_r + (G - TMJ) * 2048, KK)
                              : frag_kmajor(sr, kfrag[KK], wm * WM + (G - TMJ) * 32);
  }
  template <int KK, int M>
  __device__ __forceinline__ void load(int kt, Frags& f) const {
    if constexpr (frag_on(0)) load_one<KK, 0, M>(kt, f);
    if constexpr (frag_on(1)) load_one<KK, 1, M>(kt, f);
    if constexpr (frag_on(2)) load_one<KK, 2, M>(kt, f);
    if constexpr (frag_on(3)) load_one<KK, 3, M>(kt, f);
    if constexpr (frag_on(4)) load_one<KK, 4, M>(kt, f);
    if constexpr (frag_on(5)) load_one<KK, 5, M>(kt, f);
  }

  // Identity term of slice kt, which crosses this wave's identity at tile F:
  // acc[i][F] += v A[r][k], k = the accumulator column, from the A slice in K
  // form (byte r*64 + ((k/8) ^ ((r/4)%4))*16 + (k%8)*2, the same chunk order
  // for the four rows r of a read).  The accumulator of a 32 x 32 tile holds,
  // in lane l, column l%32 and rows 8q + 4(l/32) + e (value 4q + e);
  // ds_read_b64_tr_b16 gives lane l of a 16-lane group the four values of one
  // column in four consecutive rows, so one read per q delivers the lane's
  // four rows.
  template <int F, int I0 = 0, int I1 = TMI>
  __device__ __forceinline__ void ident_add(int kt, f32x16 (&acc)[TMI][TMJ]) const {
    static_assert(IDENT == IDENT_COL, "the column identity is the only one");
    const int l16 = lane & 15, g = lane >> 4;
    const int k16 = 16 * (g & 1) + 4 * (l16 & 3);  // first column of the lane's 8-byte chunk
    // The read of rows rb = wm WM + 32 i + 8 q + 4 (g/2) + l16/4 sits at
    // base + (32 i + 8 q) 64 + ((k16/8) ^ ((rb/4) % 4)) 16, and (rb/4) % 4 =
    // (2 q + g/2) % 4 only depends on q's parity: two per-lane bases, the rest
    // an immediate offset of the read.
    const int rlane = wm * WM + 4 * (g >> 1) + (l16 >> 2);
    const uint32_t base = uint32_t(rlane * 64 + (k16 & 7) * 2);
    const uint32_t b0 = base + uint32_t(((k16 >> 3) ^ ((g >> 1) & 3)) << 4);
    const uint32_t b1 = base + uint32_t(((k16 >> 3) ^ ((2 + (g >> 1)) & 3)) << 4);
    {
      const char* sr = reinterpret_cast<const char*>(rslot(kt));
#pragma unroll
      for (int i = I0; i < I1; ++i)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          if (!tile_on(i, F)) continue;
          const uint32_t off = ((q & 1) ? b1 : b0) + uint32_t((32 * i + 8 * q) * 64);
          const i16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(sr + off));
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[i][F][4 * q + e] = fmaf(id_v, bf2f(uint16_t(v[e])), acc[i][F][4 * q + e]);
        }
    }
  }

  // Step kt: slice kt is consumed in form M, slice kt+1 (its k step 0 fragments)
  // is read in form MN, and slice kt+NSTAGE-1 is loaded in form RF (RF < 0:
  // decided from its index).  Fragments ping-pong at half-slice granularity: the k
  // step 1 reads of slice kt go out one per MFMA of its k step 0, and (after
  // the slice-kt+1 barrier) the k step 0 reads of slice kt+1 one per MFMA of
  // the k step 1.  At the barrier of step kt every wave has consumed slice
  // kt-1, so its slot takes slice kt+NSTAGE-1; those direct loads are
  // interleaved one by one with the k step 1 MFMAs as well.  F >= 0: the
  // slice crosses this wave's identity at tile F (ident_add).
  template <int M, int MN, int F, int RF = -1, int G = -1>
  __device__ __forceinline__ void body(int kt, Frags& fa, Frags& fb, f32x16 (&acc)[TMI][TMJ]) const {
    static_assert(TMI * TMJ == 8 && SLICE_DMA <= 8 && TMI + TMJ <= 8, "one read / direct load per MFMA");
#define MMUON_MFMA(f, g)                                                                          \
    if constexpr (tile_on((g) / TMJ, (g) % TMJ))                                                  \
      acc[(g) / TMJ][(g) % TMJ] = mfma(f.r[(g) / TMJ], f.c[(g) % TMJ], acc[(g) / TMJ][(g) % TMJ]);
#define MMUON_STEP0(g)                                                           \
    MMUON_MFMA(fa, g)                                                            \
    if constexpr ((g) < TMI + TMJ && frag_on(g)) load_one<1, (g), M>(kt, fb);    \
    __builtin_amdgcn_sched_barrier(0);
    MMUON_STEP0(0) MMUON_STEP0(1) MMUON_STEP0(2) MMUON_STEP0(3)
    MMUON_STEP0(4) MMUON_STEP0(5) MMUON_STEP0(6) MMUON_STEP0(7)
#undef MMUON_STEP0
    // G >= 0: the second half of the identity term of slice kt-1 (tile G), whose
    // slot is refilled only after this step's barrier
    if constexpr (G >= 0) ident_add<G, TMI / 2, TMI>(kt - 1, acc);
    wait_vm<(NSTAGE - 3) * DMA>();  // slice kt+1; the later ones may stay in flight
    barrier();
    // on the last step slice kt+1 does not exist and the reads of its slot go
    // unused; near the end a consumed slot is refilled with slice KT-1 so every
    // step has the same shape
    const int src = kt + NSTAGE - 1 < KT ? kt + NSTAGE - 1 : KT - 1;
    const int slot = kt + NSTAGE - 1;
#define MMUON_STEP1(g)                                                               \
    MMUON_MFMA(fb, g)                                                                \
    if constexpr ((g) < TMI + TMJ && frag_on(g)) load_one<0, (g), MN>(kt + 1, fa);   \
    if constexpr ((g) < DMA) issue_one<(g), RF>(src, slot);                          \
    __builtin_amdgcn_sched_barrier(0);
    // Raised wave priority from the barrier to the end of k step 1: a wave
    // still in this phase (reads of slice kt+1, direct loads) wins issue over
    // the SIMD's other wave once that one has moved on to the next step's
    // k step 0, so the wave behind catches up before the next barrier
    // (measured: Newton-Schulz 1-2% faster on the 6.89B groups).
    __builtin_amdgcn_s_setprio(1);
    MMUON_STEP1(0) MMUON_STEP1(1) MMUON_STEP1(2) MMUON_STEP1(3)
    MMUON_STEP1(4) MMUON_STEP1(5) MMUON_STEP1(6) MMUON_STEP1(7)
#undef MMUON_STEP1
#undef MMUON_MFMA
    __builtin_amdgcn_s_setprio(0);
    // the first half of slice kt's identity term (the slot of slice kt is
    // refilled only after the next barrier)
    if constexpr (F >= 0) ident_add<F, 0, TMI / 2>(kt, acc);
  }

  // Slices a .. b-1 in form M (b > a), the last of them reading slice b in form
  // MN.  Runs start and end at multiples of BM / BK = 8 slices, so the slices the
  // last NSTAGE - 1 steps load lie in the next run (form MN) and every load's
  // form is known at compile time.
  static_assert(BM / BK >= NSTAGE - 1, "a run is longer than the loads in flight");
  template <int M, int MN>
  __device__ __forceinline__ void run_span(int a, int b, Frags& fa, Frags& fb, f32x16 (&acc)[TMI][TMJ]) const {
    int kt = a;
    for (; kt < b - (NSTAGE - 1); ++kt) body<M, M, -1, M>(kt, fa, fb, acc);
    for (; kt < b - 1; ++kt) body<M, M, -1, MN>(kt, fa, fb, acc);
    body<M, MN, -1, MN>(b - 1, fa, fb, acc);
  }

  __device__ __forceinline__ void run(f32x16 (&acc)[TMI][TMJ]) const {
#pragma unroll
    for (int i = 0; i < TMI; ++i)
#pragma unroll
      for (int j = 0; j < TMJ; ++j) acc[i][j] = f32x16{};
    // slice runs: TT [0, t1), KT [t1, t2), then ML to the end
    const int t1 = RK == OP_SPLIT ? thr_r : 0;
    const int t2 = CK == OP_SPLIT ? thr_c : (CK == OP_T ? t1 : 0);
    // slices 0 .. NSTAGE-2 (beyond the last slice: refills with slice KT-1)
#pragma unroll
    for (int q = 0; q < NSTAGE - 1; ++q) issue(q < KT ? q : KT - 1, q);
    wait_vm<(NSTAGE - 2) * DMA>();  // slice 0 visible, the others may stay in flight
    barrier();
    Frags fa, fb;
    if (t1 > 0) load<0, M_TT>(0, fa);
    else if (CK == OP_SPLIT && t2 > 0) load<0, M_KT>(0, fa);
    else load<0, ML>(0, fa);
    if constexpr (RK == OP_SPLIT) {
      if (t1 > 0) {
        if (CK == OP_SPLIT && t2 == t1) run_span<M_TT, M_KK>(0, t1, fa, fb, acc);
        else run_span<M_TT, M_KT>(0, t1, fa, fb, acc);
      }
    }
    if constexpr (CK == OP_SPLIT) {
      if (t2 > t1) run_span<M_KT, M_KK>(t1, t2, fa, fb, acc);
    }
    // the last run (every remaining slice in form ML), with the identity steps
    const int k0 = t2;
    // every slice this run loads is in form ML
    if constexpr (IDENT == IDENT_NONE) {
      for (int kt = k0; kt < KT; ++kt) body<ML, ML, -1, ML>(kt, fa, fb, acc);
    } else {
      // the slices starting at diag0 cross this wave's identity tiles in
      // order (diag0 is a multiple of the wave's extent along K and lies in
      // the last run)
      static_assert(TMJ == 2, "a wave's identity columns span two slices");
      const int kd = diag0 / BK;
      for (int kt = k0; kt < kd; ++kt) body<ML, ML, -1, ML>(kt, fa, fb, acc);
      body<ML, ML, 0, ML>(kd, fa, fb, acc);
      body<ML, ML, 1, ML, 0>(kd + 1, fa, fb, acc);
      if (kd + TMJ < KT) {
        body<ML, ML, -1, ML, 1>(kd + TMJ, fa, fb, acc);
        for (int kt = kd + TMJ + 1; kt < KT; ++kt) body<ML, ML, -1, ML>(kt, fa, fb, acc);
      } else {
        // the last slice crossed the identity; the final refills go to other slots
        ident_add<1, TMI / 2, TMI>(KT - 1, acc);
      }
    }
    wait_vm<0>();  // the refills of the last two steps land before the ring is reused
  }
};

// Wave plan of a diagonal tile of a symmetric product.  Only its 36 32 x 32
// MFMA tiles on or above the diagonal (R <= C, units of 32 rows / columns) are
// computed; they are dealt to the 8 waves so that the two waves of every SIMD
// (waves w and w + 4) hold 9 between them, against 16 per SIMD in a full tile.
// Wave w computes, inside the 128 x 64 window (vwm, vwn) of the regular wave
// grid (rows 128 vwm.., columns 64 vwn..), the 32 x 32 tiles of its mask
// (bit i * TMJ + j: window tile row i, column j):
//   w0 (0,2) all 8      w4 (0,1) tile (3,1) = (R 3, C 3)
//   w1 (0,3) all 8      w5 (1,3) tile (3,1) = (R 7, C 7)
//   w2 (0,0) j >= i: 3  w6 (0,1) rows 0-2: 6
//   w3 (1,2) j >= i: 3  w7 (1,3) rows 0-2: 6
// Every tile on or above the diagonal is computed by exactly one wave and no
// tile below it by any; the staging fills those from their transposes.
constexpr int mask_upper() {
  int m = 0;
  for (int i = 0; i < TMI; ++i)
    for (int j = 0; j < TMJ; ++j)
      if (j >= i) m |= 1 << (i * TMJ + j);
  return m;
}
constexpr int MASK_FULL = 0xFF;
constexpr int MASK_UPPER = mask_upper();        // (0,0), (0,1), (1,1)
constexpr int MASK_LAST = 1 << (3 * TMJ + 1);   // (3,1)
constexpr int MASK_FIRST6 = (1 << (3 * TMJ)) - 1;  // rows 0-2
static_assert(TMI == 4 && TMJ == 2 && BM == 8 * 32 && WM == 4 * 32 && WN == 2 * 32,
              "the plan deals the 8 x 8 grid of 32 x 32 tiles of a 256 x 256 tile");

struct WavePlan {
  int vwm, vwn, mask;
};
__device__ __forceinline__ WavePlan diag_plan(int wave) {
  switch (wave) {
    case 0: return {0, 2, MASK_FULL};
    case 1: return {0, 3, MASK_FULL};
    case 2: return {0, 0, MASK_UPPER};
    case 3: return {1, 2, MASK_UPPER};
    case 4: return {0, 1, MASK_LAST};
    case 5: return {1, 3, MASK_LAST};
    case 6: return {0, 1, MASK_FIRST6};
    default: return {1, 3, MASK_FIRST6};
  }
}
// Full tile: the 2 x 4 grid of 128 x 64 windows, the two waves of one column
// window (wave 2 wn and 2 wn + 1) on different SIMDs (a SIMD runs waves w and
// w + 4): a K slice that crosses a window's identity columns (POLY) then
// gives each SIMD one wave of identity work beside its other wave's MFMAs,
// instead of both of one SIMD's waves while the others wait at the barrier.
__device__ __forceinline__ WavePlan full_plan(int wave) { return {wave & 1, wave >> 1, MASK_FULL}; }

template <int RK, int CK, int IDENT, int MASK, bool SHARED>
__device__ __forceinline__ void mainloop_run(const uint16_t* rsrc_k, const uint16_t* rsrc_t, int thr_r,
                                             const uint16_t* csrc_k, const uint16_t* csrc_t, int thr_c,
                                             int64_t pstride, int KT, uint16_t* lds, f32x16 (&acc)[TMI][TMJ],
                                             float ident_v, int diag, int vwm, int vwn) {
  Pipe<RK, CK, IDENT, MASK, SHARED> p;
  p.rsrc_k = rsrc_k;
  p.rsrc_t = rsrc_t;
  p.csrc_k = csrc_k;
  p.csrc_t = csrc_t;
  p.thr_r = thr_r;
  p.thr_c = thr_c;
  p.pstride_b = uint32_t(pstride) * 2;
  p.KT = KT;
  p.lane = threadIdx.x & 63;
  p.wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // its share of the direct loads
  p.wm = vwm;                                                 // its window of the output tile
  p.wn = vwn;
  p.lds = lds;
  p.lds0 = lds_addr(lds);
  p.k_loff = kmajor_lane_offset(p.lane);
#pragma unroll
  for (int kk = 0; kk < BK / 16; ++kk) p.kfrag[kk] = kmajor_frag_base(kk, p.lane);
  p.tfrag_r = rowmajor_frag_base(p.wm * TMI, p.lane);
  p.tfrag_c = rowmajor_frag_base(p.wn * TMJ, p.lane);
  p.diag0 = diag + p.wn * WN;
  p.id_v = ident_v;
  p.run(acc);
}

// Operand sources: *_k the K form (panel 0 at the operand's first row), *_t the
// T form (row 0 of the first panel holding the operand's rows); thr_*: slices
// kt < thr are T (OP_SPLIT); pstride: elements per panel.  ident_v: the identity
// scalar; diag: K index of the tile's first column (IDENT_COL).
// sym_diag (workgroup-uniform): a diagonal tile of a symmetric product, whose
// work is dealt by diag_plan; SHARE: its row and column operands are the same
// rows (SYRK, POLY: loaded once, Pipe SHARED), else two stacks' bands of the
// same rows (SYMM).  idle (wave-uniform, full tiles only): the wave's window
// holds only zero padding columns; it issues its share of the direct loads and
// leaves its accumulators zero.
template <int RK, int CK, int IDENT = IDENT_NONE, bool SHARE = true>
__device__ __forceinline__ void mainloop(const uint16_t* rsrc_k, const uint16_t* rsrc_t, int thr_r,
                                         const uint16_t* csrc_k, const uint16_t* csrc_t, int thr_c,
                                         int64_t pstride, int KT, uint16_t* lds, f32x16 (&acc)[TMI][TMJ],
                                         float ident_v = 0.f, int diag = 0, bool sym_diag = false,
                                         bool idle = false) {
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const WavePlan plan = sym_diag ? diag_plan(wave) : full_plan(wave);
#define MMUON_RUN(MASK, SH)                                                                                  \
  mainloop_run<RK, CK, IDENT, MASK, SH>(rsrc_k, rsrc_t, thr_r, csrc_k, csrc_t, thr_c, pstride, KT, lds, acc, \
                                        ident_v, diag, plan.vwm, plan.vwn)
  if (!sym_diag && idle) MMUON_RUN(0, false);
  else if (!sym_diag) MMUON_RUN(MASK_FULL, false);
  else if (plan.mask == MASK_FULL) MMUON_RUN(MASK_FULL, SHARE);
  else if (plan.mask == MASK_UPPER) MMUON_RUN(MASK_UPPER, SHARE);
  else if (plan.mask == MASK_LAST) MMUON_RUN(MASK_LAST, SHARE);
  else MMUON_RUN(MASK_FIRST6, SHARE);
#undef MMUON_RUN
}

// D[i][j] accumulators of this wave -> T[j][i] in the staging area, each value
// scaled by f before the bf16 rounding.  Lane geometry: the lane holds column
// j = 64 wn + 32 tj + lane%32 and rows i = 128 wm + 32 ti + 8 qg + 4 (lane/32) + e,
// (wm, wn) the wave's window.  diag: a diagonal tile of a symmetric product
// computed by diag_plan; every computed tile above the diagonal also fills its
// mirror below it, T[i][j] = D[i][j] (copied from the staged tile), and so does
// the upper triangle of each 32 x 32 tile on the diagonal (written after, and
// so replacing, the values the lane pairs computed below it: equal bits when
// both operands are one symmetric matrix, rounding-level apart for SYMM's two
// commuting ones); its diagonal entries i = j < dlim get dadd added (in fp32,
// before the rounding).
__device__ __forceinline__ void stage_tile(char* stage, const f32x16 (&acc)[TMI][TMJ], float f,
                                           bool diag = false, float dadd = 0.f, int dlim = 0) {
  const int tid = fresh_tid();
  const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const WavePlan plan = diag ? diag_plan(wave) : full_plan(wave);
  const int wm = plan.vwm, wn = plan.vwn;
#pragma unroll
  for (int i = 0; i < TMI; ++i) {
#pragma unroll
    for (int j = 0; j < TMJ; ++j) {
      const int R = wm * (WM / 32) + i, C = wn * (WN / 32) + j;
      if (!((plan.mask >> (i * TMJ + j)) & 1)) continue;
#pragma unroll
      for (int qg = 0; qg < 4; ++qg) {
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = f * acc[i][j][qg * 4 + e];
        if (diag && R == C) {
          // the 32 x 32 tile on the diagonal: lane l holds entry (l%32, l%32)
          // at qg = (l%32)/8, e = l%8 - 4 (l/32) when that lies in [0, 4)
          const int d = lane & 31, e = (d & 7) - 4 * (lane >> 5);
          if ((d >> 3) == qg && e >= 0 && e < 4 && 32 * R + d < dlim) {
#pragma unroll
            for (int x = 0; x < 4; ++x)
              if (x == e) v[x] += dadd;
          }
        }
        const int row = wn * WN + j * 32 + (lane & 31);
        const int col = wm * WM + i * 32 + qg * 8 + (lane >> 5) * 4;
        *reinterpret_cast<uint2*>(stage + tile_off(row, col)) = make_uint2(f2bf2(v[0], v[1]), f2bf2(v[2], v[3]));
      }
      if (diag && C == R) {
        // a 32 x 32 tile on the diagonal: its upper triangle replaces the
        // values just staged below it
#pragma unroll
        for (int qg = 0; qg < 4; ++qg)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int row = wm * WM + i * 32 + qg * 8 + (lane >> 5) * 4 + e;
            const int col = wn * WN + j * 32 + (lane & 31);
            if (row < col) *reinterpret_cast<uint16_t*>(stage + tile_off(row, col)) = f2bf(f * acc[i][j][qg * 4 + e]);
          }
      }
    }
  }
  if (!diag) return;
  // The mirrors of this wave's tiles above the diagonal (C > R): the tile it
  // has just staged, T[32C + r][32R + i] = D[32R + i][32C + r], read
  // transposed (ds_read_b64_tr_b16, as stage_cols reads) gives rows of D,
  // stored as 16-B chunks at T[32R + i][32C + r] -- four reads and two writes
  // per lane and tile, the staged bf16 values copied bit for bit.  The wave's
  // LDS operations complete in order, and no other wave writes or reads
  // either region.
  asm volatile("" ::: "memory");
  const int l16 = lane & 15, grp = lane >> 4;
#pragma unroll
  for (int i = 0; i < TMI; ++i) {
#pragma unroll
    for (int j = 0; j < TMJ; ++j) {
      const int R = wm * (WM / 32) + i, C = wn * (WN / 32) + j;
      if (!((plan.mask >> (i * TMJ + j)) & 1) || C <= R) continue;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int r0 = 32 * C + grp * 8, i0 = 32 * R + 16 * h;
        const int tr = r0 + (l16 >> 2), tc = i0 + ((l16 & 3) << 2);
        const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(stage + tile_off(tr, tc)));
        const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(stage + tile_off(tr + 4, tc)));
        uint4 v;
        v.x = uint32_t(uint16_t(lo[0])) | (uint32_t(uint16_t(lo[1])) << 16);
        v.y = uint32_t(uint16_t(lo[2])) | (uint32_t(uint16_t(lo[3])) << 16);
        v.z = uint32_t(uint16_t(hi[0])) | (uint32_t(uint16_t(hi[1])) << 16);
        v.w = uint32_t(uint16_t(hi[2])) | (uint32_t(uint16_t(hi[3])) << 16);
        *reinterpret_cast<uint4*>(stage + tile_off(i0 + l16, r0)) = v;
      }
    }
  }
}

// Staged rows -> a panel-layout destination with the same rows: dst[r][i] =
// T[r][i] for the BN staged rows, dst at the first staged row of the tile's
// first column panel (panel stride pstride).  One wave instruction writes rows
// 16u .. 16u+15 of one panel (1 KiB contiguous).
__device__ __forceinline__ void stage_rows(const char* stage, uint16_t* dst, int64_t pstride) {
  const int tid = fresh_tid();
  const int lane = tid & 63, wave = tid >> 6;
#pragma unroll 4
  for (int it = 0; it < 8 * (BN / 16) / NWAVES; ++it) {
    const int u = wave + NWAVES * it;  // 8 panels x BN/16 row blocks
    const int q = u & 7, r = (u >> 3) * 16 + (lane >> 2);
    const int i = q * 32 + (lane & 3) * 8;
    const uint4 v = *reinterpret_cast<const uint4*>(stage + tile_off(r, i));
    *reinterpret_cast<uint4*>(dst + q * pstride + r * PANEL + (lane & 3) * 8) = v;
  }
}

// Staged columns -> rows of the destination: dst[i][r] = T[r][i] (256 rows i,
// BN columns r).  ds_read_b64_tr_b16 (16-lane groups): lane l of a group
// addresses T row r0 + l/4 at column i0 + 4*(l%4) and receives T[r0..r0+3][i0 + l];
// two reads give 8 consecutive r of destination row i0 + l.  The four groups of
// a wave take consecutive 8-column chunks, so one wave instruction covers
// destination rows i0 .. i0+15, columns 32t .. 32t+31: one panel's contiguous
// 1 KiB.  `fn(i, r, uint4)` consumes destination row i, columns r..r+7.
template <class Fn>
__device__ __forceinline__ void stage_cols(const char* stage, Fn&& fn) {
  const int tid = fresh_tid();
  const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15, grp = lane >> 4;
#pragma unroll 2
  for (int it = 0; it < 16 * (BN / 32) / NWAVES; ++it) {
    const int task = wave + NWAVES * it;
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
// SYRK / POLY / SYMM: symmetric m x m outputs of which only the 256 x 256
// tiles on and above the diagonal are computed and stored (tile ti x tc,
// tc >= ti; a diagonal tile in full).  SYRK reads X (K form); POLY reads the
// stored upper tiles of A (operand band R: T form left of its diagonal block,
// K form from there on); SYMM (C = S1 S2 of two symmetric stacks that commute,
// as polynomials in one Gram matrix do, so C is symmetric) reads its row band
// from S1 and its column band from S2 in the same way.
// ---------------------------------------------------------------------------
static_assert(BM == BN, "square tiles: a symmetric tile is either diagonal or strictly upper");
template <int STAGE>
__device__ __forceinline__ void sym_work(const NsArgs& a, uint16_t* lds, int v) {
  const int nt = a.mp / BM, nc = a.mp / BN;
  const int tiles = nt * nc - R_SYM * nt * (nt - 1) / 2;
  int b, t;
  if (!decode_tile(v, tiles, a.N, b, t)) return;
  int ti, tc;
  sym_tile(t, nc, ti, tc);

  const uint16_t* src;
  int K;
  if (STAGE == NS_SYRK) {
    src = static_cast<const uint16_t*>(a.x_in) + int64_t(b) * a.mp * a.np;
    K = a.kx;
  } else {
    src = static_cast<const uint16_t*>(a.a_in) + int64_t(b) * a.mp * a.mp;
    K = a.mp;
  }
  // SYMM: the column operand's stack (POLY: the row operand's own)
  const uint16_t* src2 = STAGE == NS_SYMM ? static_cast<const uint16_t*>(a.b_in) + int64_t(b) * a.mp * a.mp : src;
  const int64_t pstride = int64_t(a.mp) * PANEL;
  const int r0 = ti * BM, c0 = tc * BN;
  // on a diagonal tile only the 32 x 32 tiles on or above the diagonal are
  // computed; the others are staged from their transposes
  const bool diag = tc == ti;
  f32x16 acc[TMI][TMJ];
  if (STAGE == NS_SYRK)
    mainloop<OP_K, OP_K>(src + r0 * PANEL, nullptr, 0, src + c0 * PANEL, nullptr, 0, pstride, K / BK, lds, acc,
                         0.f, 0, diag);
  else if (STAGE == NS_POLY)  // acc = A A + (b/c) A, so P = c acc + a I = a I + b A + c A A
    mainloop<OP_SPLIT, OP_SPLIT, IDENT_COL>(src + r0 * PANEL, src + (r0 / PANEL) * pstride, r0 / BK,
                                            src + c0 * PANEL, src + (c0 / PANEL) * pstride, c0 / BK,
                                            pstride, K / BK, lds, acc, a.cb / a.cc, c0, diag);
  else  // SYMM: acc = S1 S2; a diagonal tile loads both operands' bands
    mainloop<OP_SPLIT, OP_SPLIT, IDENT_NONE, false>(src + r0 * PANEL, src + (r0 / PANEL) * pstride, r0 / BK,
                                                    src2 + c0 * PANEL, src2 + (c0 / PANEL) * pstride, c0 / BK,
                                                    pstride, K / BK, lds, acc, 0.f, 0, diag);

  float f = STAGE == NS_POLY ? a.cc : 1.f;  // SYRK: s^2 on the first iteration
  if (STAGE == NS_SYRK && a.scale != nullptr) {
    const float s = a.scale[b];
    f = s * s;
  }
  uint16_t* out = static_cast<uint16_t*>(a.out) + int64_t(b) * a.mp * a.mp;
  char* stage = reinterpret_cast<char*>(lds);
  barrier();  // every wave is done with the ring
  // POLY: a on the diagonal of the m valid rows (the padding stays zero)
  stage_tile(stage, acc, f, diag, STAGE == NS_POLY ? a.ca : 0.f, STAGE == NS_POLY ? a.m - r0 : 0);
  barrier();
  if (!diag) {
    // upper tile C[r0 + i][c0 + r] = T[r][i]
    uint16_t* dst = out + (c0 / PANEL) * pstride + int64_t(r0) * PANEL;
    stage_cols(stage, [&](int i, int r, const uint4& u) {
      *reinterpret_cast<uint4*>(dst + (r >> 5) * pstride + i * PANEL + (r & 31)) = u;
    });
  } else {
    // diagonal tile in full, through its mirror C[r0 + r][r0 + i] = T[r][i]
    stage_rows(stage, out + (r0 / PANEL) * pstride + int64_t(r0) * PANEL, pstride);
  }
}

template <int STAGE>
__global__ __launch_bounds__(NT, WG_PER_CU) void ns_sym_bf16(NsArgs a, int total) {
  __shared__ __attribute__((aligned(1024))) uint16_t lds[LDS_ELEMS];
  for (int v = blockIdx.x; v < total; v += gridDim.x) {
    sym_work<STAGE>(a, lds, v);
    barrier();  // the staging area is read before the next tile's loads refill the ring
  }
}

// ---------------------------------------------------------------------------
// PX / PX_APPLY: X' = s P X (P = a I + b A + c A A from POLY), m x n output
// tile (256 x 256), K = m.  D[i][j] in registers (lane holds column j, rows
// i..i+3).  T[j][i] = X'[r0 + i][c0 + j] is staged in LDS;
// X' rows (PX, and the parameter rows of an untransposed block) are T's
// columns, the parameter rows of a tall block (param[j][i]) are T's rows.
// ---------------------------------------------------------------------------

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
__device__ __forceinline__ void px_work(const NsArgs& a, uint16_t* lds, int v) {
  const int tiles_i = a.mp / BM;
  const int tiles = tiles_i * (a.np / BN);
  int b, t;
  if (!decode_tile(v, tiles, a.N, b, t)) return;
  // column-band-major: the tiles_i tiles that read one column band of X are
  // consecutive virtual tiles, so they run in the same round on one XCD
  // whenever tiles_i divides the workgroups one XCD runs per round (32 on 256
  // CUs; m <= 1024 at every model size here) and the band is fetched from HBM
  // once.  A block with more tiles than a round (n = 2752: 44) is split
  // between rounds at a column-band boundary, so only its P row bands, the
  // smaller operand, are fetched twice.
  const int tc = t / tiles_i, ti = t % tiles_i;
  const int r0 = ti * BM, c0 = tc * BN;

  const int64_t pstride = int64_t(a.mp) * PANEL;
  const uint16_t* P = static_cast<const uint16_t*>(a.a_in) + int64_t(b) * a.mp * a.mp;
  const uint16_t* X = static_cast<const uint16_t*>(a.x_in) + int64_t(b) * a.mp * a.np + (c0 / PANEL) * pstride;
  f32x16 acc[TMI][TMJ];
  // acc = P X; a wave whose 64 columns all lie in the zero padding (n <= column
  // < np) computes nothing: its part of X' stays zero
  const int wn = full_plan(__builtin_amdgcn_readfirstlane(threadIdx.x >> 6)).vwn;
  mainloop<OP_SPLIT, OP_T>(P + r0 * PANEL, P + (r0 / PANEL) * pstride, r0 / BK, nullptr, X, 0, pstride, a.mp / BK,
                           lds, acc, 0.f, 0, false, c0 + wn * WN >= a.n);

  const float s = a.scale != nullptr ? a.scale[b] : 1.f;
  char* stage = reinterpret_cast<char*>(lds);
  // apply: param += alpha * u; the parameter block is stored (m x n)
  // untransposed or (n x m) for a tall block
  auto* prm = STAGE == NS_PX_APPLY ? reinterpret_cast<typename TP::storage*>(a.blocks[b].param) : nullptr;
  const int m = a.m, n = a.n;
  // 16-B vector access: aligned blocks and a row length that keeps chunks aligned
  const bool vec = a.vec && ((TRANS ? m : n) % 8 == 0);
  // bf16 parameters, tile inside the block: every parameter chunk of this
  // thread is loaded in batches ahead of its use (the first batch before the
  // tile is staged), then combined and stored
  constexpr bool BF16P = sizeof(typename TP::storage) == 2;
  const bool fast = STAGE == NS_PX_APPLY && BF16P && vec && r0 + BM <= m && c0 + BN <= n;
  constexpr int CH = BN * BM / 8 / NT;  // 16-B chunks per thread
  constexpr int BATCH = 8;
  const int tid = fresh_tid();
  const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15, grp = lane >> 4;
  // chunk q of this thread: parameter offset, staged row r and column c of
  // its first element (TRANS: 8 consecutive staged columns; else 8 staged rows)
  auto chunk = [&](int q, int& r, int& c) -> int64_t {
    if (TRANS) {
      r = q * (NT / 32) + (tid >> 5);
      c = (tid & 31) * 8;
      return int64_t(c0 + r) * m + r0 + c;
    }
    const int task = wave + NWAVES * q;  // the stage_cols mapping
    c = (task & 15) * 16;                // i0
    r = (task >> 4) * 32 + grp * 8;
    return int64_t(r0 + c + l16) * n + c0 + r;
  };
  uint4 pv[BATCH];
  if constexpr (STAGE == NS_PX_APPLY && BF16P) {
    if (fast) {
#pragma unroll
      for (int q = 0; q < BATCH; ++q) {
        int r, c;
        pv[q] = *reinterpret_cast<const uint4*>(prm + chunk(q, r, c));
      }
    }
  }
  barrier();  // every wave is done with the ring
  stage_tile(stage, acc, s);
  barrier();
  if (STAGE == NS_PX) {
    // X'[r0 + i][c0 + r] = T[r][i]
    uint16_t* dst = static_cast<uint16_t*>(a.out) + int64_t(b) * a.mp * a.np + (c0 / PANEL) * pstride +
                    int64_t(r0) * PANEL;
    stage_cols(stage, [&](int i, int r, const uint4& u) {
      *reinterpret_cast<uint4*>(dst + (r >> 5) * pstride + i * PANEL + (r & 31)) = u;
    });
    return;
  }
  const float alpha = a.alpha;
  if constexpr (BF16P) {
    if (fast) {
#pragma unroll
      for (int q0 = 0; q0 < CH; q0 += BATCH) {
        if (q0 > 0) {
#pragma unroll
          for (int q = 0; q < BATCH; ++q) {
            int r, c;
            pv[q] = *reinterpret_cast<const uint4*>(prm + chunk(q0 + q, r, c));
          }
        }
#pragma unroll
        for (int q = 0; q < BATCH; ++q) {
          int r, c;
          const int64_t o = chunk(q0 + q, r, c);
          uint4 u;
          if (TRANS) {
            u = *reinterpret_cast<const uint4*>(stage + tile_off(r, c));
          } else {
            const int tr = r + (l16 >> 2), tc = c + ((l16 & 3) << 2);
            const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(stage + tile_off(tr, tc)));
            const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(stage + tile_off(tr + 4, tc)));
            u.x = uint32_t(uint16_t(lo[0])) | (uint32_t(uint16_t(lo[1])) << 16);
            u.y = uint32_t(uint16_t(lo[2])) | (uint32_t(uint16_t(lo[3])) << 16);
            u.z = uint32_t(uint16_t(hi[0])) | (uint32_t(uint16_t(hi[1])) << 16);
            u.w = uint32_t(uint16_t(hi[2])) | (uint32_t(uint16_t(hi[3])) << 16);
          }
          const uint32_t w[4] = {u.x, u.y, u.z, u.w};
          uint32_t pw[4] = {pv[q].x, pv[q].y, pv[q].z, pv[q].w};
#pragma unroll
          for (int h = 0; h < 4; ++h) {
            const float u0 = __uint_as_float(w[h] << 16), u1 = __uint_as_float(w[h] & 0xffff0000u);
            const float p0 = __uint_as_float(pw[h] << 16), p1 = __uint_as_float(pw[h] & 0xffff0000u);
            pw[h] = f2bf2(fmaf(alpha, u0, p0), fmaf(alpha, u1, p1));
          }
          *reinterpret_cast<uint4*>(prm + o) = make_uint4(pw[0], pw[1], pw[2], pw[3]);
        }
      }
      return;
    }
  }
  if (TRANS) {
    const int c = (tid & 31) * 8;
    for (int q = 0; q < BN / (NT / 32); ++q) {
      const int r = q * (NT / 32) + (tid >> 5);  // staged row = X' column = parameter row
      const int pr = c0 + r, pc = r0 + c;
      if (pr >= n || pc >= m) continue;
      const uint4 u8 = *reinterpret_cast<const uint4*>(stage + tile_off(r, c));
      apply_chunk<TP>(prm, int64_t(pr) * m + pc, u8, alpha, min(8, m - pc), vec);
    }
  } else {
    stage_cols(stage, [&](int i, int r, const uint4& u) {
      const int pr = r0 + i, pc = c0 + r;
      if (pr < m && pc < n) apply_chunk<TP>(prm, int64_t(pr) * n + pc, u, alpha, min(8, n - pc), vec);
    });
  }
}

template <int STAGE, bool TRANS, class TP>
__global__ __launch_bounds__(NT, WG_PER_CU) void ns_px_bf16(NsArgs a, int total) {
  __shared__ __attribute__((aligned(1024))) uint16_t lds[LDS_ELEMS];
  for (int v = blockIdx.x; v < total; v += gridDim.x) {
    px_work<STAGE, TRANS, TP>(a, lds, v);
    barrier();  // the staging area is read before the next tile's loads refill the ring
  }
}

// ---------------------------------------------------------------------------
// fp32 Newton-Schulz (the pretrain copy keeps the buffer dtype) on the fp32
// matrix cores (v_mfma_f32_32x32x2_f32, fp32 products and accumulation).
// 128 x 128 output tiles per 256-thread workgroup, 4 waves of 64 x 64 (2 x 2
// MFMA tiles of 32 x 32, 32 MFMAs per wave and K tile); K advances 16 per
// tile, double-buffered in LDS: the next tile's global loads (into registers)
// are in flight during the current tile's MFMAs and stored to the other buffer
// after them.  Operands reach LDS in one of two forms:
//   RK: operand rows, [row][k] (rows of X for SYRK; rows of A / P, and by
//       symmetry A's columns), 17 floats per row, so the 32 lanes that read
//       one k of 32 consecutive rows hit 32 different banks;
//   KC: [k][col] (PX's X operand, k = rows of X), 132 floats per row, 16-B
//       aligned for float4 stores.
// SYRK and POLY produce symmetric matrices: only the tiles on and above the
// diagonal are computed, each stored with its mirror (staged in LDS so both
// stores are row-contiguous), so the stored matrix is exactly symmetric.
// ---------------------------------------------------------------------------
constexpr int FT = 128;                // output tile
constexpr int FK = 16;                 // K tile
constexpr int F_NT = 256;              // 4 waves, 2 x 2
constexpr int RK_LD = FK + 1;
constexpr int KC_LD = FT + 4;
constexpr int F_OPER = FT * RK_LD;     // floats per operand buffer
static_assert(FK * KC_LD <= F_OPER, "both forms fit one operand buffer");
constexpr int F_ST = FT + 1;           // staged tile: 129 floats per row
constexpr int F_HALF = FT / 2;         // the tile is staged and stored half its rows at a time
static_assert(F_HALF * F_ST <= 4 * F_OPER, "half the staged tile fits in the operand buffers");
constexpr int F_APPLY_BATCH = 8;       // parameter elements per batch of the apply's loads
constexpr int F_RQ = FK / 4;           // float4 per operand row of a K tile
constexpr int F_QPT = FT * FK / 4 / F_NT;  // float4 per thread and operand K tile

// One operand's K tile in registers.
struct F32Stage {
  float4 v[F_QPT];
};

// rows r0 .. r0+127 of a row-major matrix (leading dimension ld), k0 .. k0+FK-1
__device__ __forceinline__ void f32_load_rows(F32Stage& g, const float* src, int64_t ld, int r0, int k0) {
#pragma unroll
  for (int j = 0; j < F_QPT; ++j) {
    const int idx = threadIdx.x + F_NT * j;
    g.v[j] = *reinterpret_cast<const float4*>(src + int64_t(r0 + idx / F_RQ) * ld + k0 + 4 * (idx % F_RQ));
  }
}
__device__ __forceinline__ void f32_store_rk(const F32Stage& g, float* s) {
#pragma unroll
  for (int j = 0; j < F_QPT; ++j) {
    const int idx = threadIdx.x + F_NT * j;
    float* d = s + (idx / F_RQ) * RK_LD + 4 * (idx % F_RQ);
    d[0] = g.v[j].x;
    d[1] = g.v[j].y;
    d[2] = g.v[j].z;
    d[3] = g.v[j].w;
  }
}
// rows k0 .. k0+FK-1 of X (leading dimension ld), columns c0 .. c0+127
__device__ __forceinline__ void f32_load_kc(F32Stage& g, const float* X, int64_t ld, int c0, int k0) {
#pragma unroll
  for (int j = 0; j < F_QPT; ++j) {
    const int idx = threadIdx.x + F_NT * j;
    g.v[j] = *reinterpret_cast<const float4*>(X + int64_t(k0 + (idx >> 5)) * ld + c0 + 4 * (idx & 31));
  }
}
__device__ __forceinline__ void f32_store_kc(const F32Stage& g, float* s) {
  // a native 4-wide vector store (a float4 struct copy here kept the staged
  // tile in scratch memory)
  typedef float f32x4_t __attribute__((ext_vector_type(4)));
#pragma unroll
  for (int j = 0; j < F_QPT; ++j) {
    const int idx = threadIdx.x + F_NT * j;
    const f32x4_t v = {g.v[j].x, g.v[j].y, g.v[j].z, g.v[j].w};
    *reinterpret_cast<f32x4_t*>(s + (idx >> 5) * KC_LD + 4 * (idx & 31)) = v;
  }
}

// Upper tile t of an nt x nt grid of tiles (ti <= tj), row-major over the
// upper triangle.
__device__ __forceinline__ void f32_sym_tile(int t, int nt, int& ti, int& tj) {
  int i = 0;
  while (t >= nt - i) {
    t -= nt - i;
    ++i;
  }
  ti = i;
  tj = i + t;
}

// Add v to the diagonal entries of an RK-form K tile in registers: rows rbase
// + 0..127 of the operand, k0 .. k0+FK-1; an element is on the diagonal when
// its row equals its k.  The quintic's linear terms enter the products this
// way: PX multiplies (P + a I) X, POLY A (A + (b/c) I); no epilogue reads
// global memory and no accumulator leaves the matrix registers.
__device__ __forceinline__ void f32_add_diag(F32Stage& g, int rbase, int k0, float v) {
#pragma unroll
  for (int j = 0; j < F_QPT; ++j) {
    const int idx = threadIdx.x + F_NT * j;
    const int d = rbase + idx / F_RQ - (k0 + 4 * (idx % F_RQ));  // row - k of the float4's first element
    if (d == 0) g.v[j].x += v;
    if (d == 1) g.v[j].y += v;
    if (d == 2) g.v[j].z += v;
    if (d == 3) g.v[j].w += v;
  }
}

// 16-deep K tiles double-buffered in 35 KiB of LDS, so four workgroups share a
// CU (three for the apply, whose epilogue holds more registers; at least three
// waves per SIMD, which hide each other's barrier and load waits: one
// workgroup per CU measured 18% slower than two, four 3% faster than two).
// The 128 x 128 output tile is staged and stored in two halves of 64 rows (the
// rows of one wave row, wr), each in the operand buffers.
template <int STAGE, class TP>
__global__ __launch_bounds__(F_NT) __attribute__((amdgpu_waves_per_eu(3))) void ns_f32(NsArgs a) {
  __shared__ __attribute__((aligned(16))) float lds[4 * F_OPER];  // [buffer 0: A, B][buffer 1: A, B]
  constexpr bool PX = STAGE == NS_PX || STAGE == NS_PX_APPLY;
  constexpr bool SYM = STAGE == NS_SYRK || STAGE == NS_POLY;
  const int b = blockIdx.y;
  int ti, tj;
  if (SYM) {
    f32_sym_tile(blockIdx.x, a.mp / FT, ti, tj);
  } else {
    const int nc = a.np / FT;
    ti = blockIdx.x / nc;
    tj = blockIdx.x % nc;
  }
  const int r0 = ti * FT, c0 = tj * FT;
  const float* X = static_cast<const float*>(a.x_in) + int64_t(b) * a.mp * a.np;
  const float* A = static_cast<const float*>(a.a_in) + int64_t(b) * a.mp * a.mp;
  const float* rsrc = STAGE == NS_SYRK ? X : A;  // rows of the row operand (and of SYRK / POLY's column operand)
  const int64_t rld = STAGE == NS_SYRK ? a.np : a.mp;
  const int K = STAGE == NS_SYRK ? a.kx : a.mp;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wr = wave >> 1, wc = wave & 1;
  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x16{};
  F32Stage ga, gb;
  const int KT = K / FK;
  f32_load_rows(ga, rsrc, rld, r0, 0);
  if (PX) f32_load_kc(gb, X, a.np, c0, 0);
  else f32_load_rows(gb, rsrc, rld, c0, 0);
  if (PX) f32_add_diag(ga, r0, 0, a.ca);
  if (STAGE == NS_POLY) f32_add_diag(gb, c0, 0, a.cb / a.cc);
  f32_store_rk(ga, lds);
  if (PX) f32_store_kc(gb, lds + F_OPER);
  else f32_store_rk(gb, lds + F_OPER);
  __syncthreads();
  for (int t = 0; t < KT; ++t) {
    const float* sa = lds + (t & 1) * 2 * F_OPER;
    const float* sb = sa + F_OPER;
    if (t + 1 < KT) {
      f32_load_rows(ga, rsrc, rld, r0, (t + 1) * FK);
      if (PX) f32_load_kc(gb, X, a.np, c0, (t + 1) * FK);
      else f32_load_rows(gb, rsrc, rld, c0, (t + 1) * FK);
    }
    // 32x32x2 steps: lane l supplies row (column) l%32 at k = 2 kk + l/32
#pragma unroll
    for (int kk = 0; kk < FK / 2; ++kk) {
      const int k = 2 * kk + (lane >> 5);
      float av[2], bv[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) av[i] = sa[(wr * 64 + i * 32 + (lane & 31)) * RK_LD + k];
#pragma unroll
      for (int j = 0; j < 2; ++j)
        bv[j] = PX ? sb[k * KC_LD + wc * 64 + j * 32 + (lane & 31)] : sb[(wc * 64 + j * 32 + (lane & 31)) * RK_LD + k];
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i], bv[j], acc[i][j], 0, 0, 0);
    }
    if (t + 1 < KT) {
      float* d = lds + ((t + 1) & 1) * 2 * F_OPER;
      if (PX) f32_add_diag(ga, r0, (t + 1) * FK, a.ca);
      if (STAGE == NS_POLY) f32_add_diag(gb, c0, (t + 1) * FK, a.cb / a.cc);
      f32_store_rk(ga, d);
      if (PX) f32_store_kc(gb, d + F_OPER);
      else f32_store_rk(gb, d + F_OPER);
    }
    __syncthreads();
  }
  const float s = a.scale != nullptr ? a.scale[b] : 1.f;
  const bool diag = SYM && tj == ti;
  float* T = lds;  // T[r - 64 h][c]: rows 64 h .. 64 h + 63 of the tile
  auto* prm = STAGE == NS_PX_APPLY ? reinterpret_cast<typename TP::storage*>(a.blocks[b].param) : nullptr;
#pragma unroll 1
  for (int h = 0; h < 2; ++h) {
    if (h) __syncthreads();  // every wave is done reading the first half
    // stage half h: accumulator value 4 q + e of MFMA tile (i, j) holds row
    // 64 wr + 32 i + 8 q + 4 (lane/32) + e, column 64 wc + 32 j + lane%32, so
    // the waves with wr == h hold the half
    if (wr == h) {
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int q = 0; q < 4; ++q)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const int r = i * 32 + 8 * q + 4 * (lane >> 5) + e, c = wc * 64 + j * 32 + (lane & 31);
              T[r * F_ST + c] = acc[i][j][4 * q + e];
            }
    }
    __syncthreads();
    // element idx of the half, two mappings (consecutive lanes along the
    // destination's rows): direct (r, c) = (64 h + idx / 128, idx % 128) and
    // mirrored (r, c) = (64 h + idx % 64, idx / 64), the latter for stores
    // along a column of the tile (a symmetric mirror, a tall block's
    // parameter rows)
    constexpr int PER = F_HALF * FT / F_NT;  // elements per thread and half
    if constexpr (SYM) {
      // SYRK: A = s^2 acc; POLY: P = c (A A + (b/c) A) = b A + c A A.  A
      // diagonal tile takes its lower triangle from the upper one: in the
      // first half from T[c][r] (c < r < 64) and, for the 64 x 64 block
      // below it, from the first half's mirror stores; in the second half
      // from T[c][r] (64 <= c < r).
      float* out = static_cast<float*>(a.out) + int64_t(b) * a.mp * a.mp;
      const float f = STAGE == NS_SYRK ? s * s : a.cc;
#pragma unroll 4
      for (int it = 0; it < PER; ++it) {
        const int idx = threadIdx.x + F_NT * it, rl = idx >> 7, c = idx & 127, r = F_HALF * h + rl;
        if (diag && c < F_HALF * h) continue;
        const float v = (diag && r > c) ? T[(c - F_HALF * h) * F_ST + r] : T[rl * F_ST + c];
        out[int64_t(r0 + r) * a.mp + c0 + c] = v * f;
      }
      if (!diag || h == 0) {
#pragma unroll 4
        for (int it = 0; it < PER; ++it) {
          const int idx = threadIdx.x + F_NT * it, rl = idx & (F_HALF - 1), c = idx / F_HALF, r = F_HALF * h + rl;
          if (diag && c < F_HALF) continue;
          out[int64_t(c0 + c) * a.mp + r0 + r] = T[rl * F_ST + c] * f;  // the mirror of (r0 + r, c0 + c)
        }
      }
    } else if constexpr (STAGE == NS_PX) {  // X' = s (a X + P X)
      float* out = static_cast<float*>(a.out) + int64_t(b) * a.mp * a.np;
#pragma unroll 4
      for (int it = 0; it < PER; ++it) {
        const int idx = threadIdx.x + F_NT * it, rl = idx >> 7, c = idx & 127;
        out[int64_t(r0 + F_HALF * h + rl) * a.np + c0 + c] = s * T[rl * F_ST + c];
      }
    } else {
      // PX_APPLY: param += alpha X' (un-transposed); the block is (m x n) or,
      // tall, (n x m).  F_APPLY_BATCH elements per batch: their parameter loads
      // are all issued before the first update is stored, so a thread waits
      // for the load latency once per batch rather than once per element.
      constexpr int PB = F_APPLY_BATCH;
      static_assert(PER % PB == 0, "whole batches per thread");
#pragma unroll 1
      for (int it0 = 0; it0 < PER; it0 += PB) {
        float pv[PB];
        int64_t off[PB];
#pragma unroll
        for (int q = 0; q < PB; ++q) {
          const int idx = threadIdx.x + F_NT * (it0 + q);
          const int rl = a.transposed ? (idx & (F_HALF - 1)) : (idx >> 7);
          const int c = a.transposed ? (idx / F_HALF) : (idx & 127);
          const int i = r0 + F_HALF * h + rl, j = c0 + c;
          off[q] = i < a.m && j < a.n ? (a.transposed ? int64_t(j) * a.m + i : int64_t(i) * a.n + j) : -1;
          pv[q] = off[q] >= 0 ? TP::load(prm, off[q]) : 0.f;
        }
#pragma unroll
        for (int q = 0; q < PB; ++q) {
          if (off[q] < 0) continue;
          const int idx = threadIdx.x + F_NT * (it0 + q);
          const int rl = a.transposed ? (idx & (F_HALF - 1)) : (idx >> 7);
          const int c = a.transposed ? (idx / F_HALF) : (idx & 127);
          TP::store(prm, off[q], fmaf(a.alpha, s * T[rl * F_ST + c], pv[q]));
        }
      }
    }
  }
}

template <int STAGE, class TP>
void launch_bf16(const NsArgs& a, hipStream_t s) {
  const int nb8 = 8 * ((a.N + 7) / 8);
  if constexpr (STAGE == NS_SYRK || STAGE == NS_POLY || STAGE == NS_SYMM) {
    const int nt = a.mp / BM;
    const int nc = a.mp / BN;
    const int total = nb8 * (nt * nc - R_SYM * nt * (nt - 1) / 2);
    hipLaunchKernelGGL((ns_sym_bf16<STAGE>), dim3(resident_grid(total)), dim3(NT), 0, s, a, total);
  } else {
    const int total = nb8 * (a.mp / BM) * (a.np / BN);
    const dim3 grid(resident_grid(total));
    if constexpr (STAGE == NS_PX) {
      hipLaunchKernelGGL((ns_px_bf16<STAGE, false, TP>), grid, dim3(NT), 0, s, a, total);
    } else {
      if (!a.transposed) hipLaunchKernelGGL((ns_px_bf16<STAGE, false, TP>), grid, dim3(NT), 0, s, a, total);
      else hipLaunchKernelGGL((ns_px_bf16<STAGE, true, TP>), grid, dim3(NT), 0, s, a, total);
    }
  }
}

template <int STAGE, class TP>
void launch_f32(const NsArgs& a, hipStream_t s) {
  const int nt = a.mp / FT;
  const int tiles = (STAGE == NS_SYRK || STAGE == NS_POLY) ? nt * (nt + 1) / 2 : nt * (a.np / FT);
  // blocks go to grid.y (at most 65535 per launch): larger stacks in chunks
  const int64_t per_x = int64_t(a.mp) * a.np, per_a = int64_t(a.mp) * a.mp;
  const int64_t per_out = (STAGE == NS_SYRK || STAGE == NS_POLY) ? per_a : per_x;
  for (int b0 = 0; b0 < a.N; b0 += 65535) {
    NsArgs c = a;
    c.N = a.N - b0 < 65535 ? a.N - b0 : 65535;
    if (a.x_in) c.x_in = static_cast<const float*>(a.x_in) + b0 * per_x;
    if (a.a_in) c.a_in = static_cast<const float*>(a.a_in) + b0 * per_a;
    if (a.out) c.out = static_cast<float*>(a.out) + b0 * per_out;
    if (a.scale) c.scale = a.scale + b0;
    if (a.blocks) c.blocks = a.blocks + b0;
    hipLaunchKernelGGL((ns_f32<STAGE, TP>), dim3(tiles, c.N), dim3(F_NT), 0, s, c);
  }
}

}  // namespace

int ns_tile_m(int ns_dtype) { return ns_dtype == MMUON_BF16 ? BM : FT; }
int ns_tile_n(int ns_dtype) { return ns_dtype == MMUON_BF16 ? 256 : FT; }  // pack tiles 256 columns
int ns_tile_k(int ns_dtype) { return ns_dtype == MMUON_BF16 ? BK : FK; }

int launch_ns_stage(const NsArgs& a, int stage, int ns_dtype, int param_dtype, hipStream_t s) {
  if (ns_dtype == MMUON_BF16) {
    switch (stage) {
      case NS_SYRK: launch_bf16<NS_SYRK, BF16T>(a, s); return 0;
      case NS_POLY: launch_bf16<NS_POLY, BF16T>(a, s); return 0;
      case NS_SYMM: launch_bf16<NS_SYMM, BF16T>(a, s); return 0;
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
