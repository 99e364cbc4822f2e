// Monarch butterfly multiply (MonarchLinear.forward_matmul) and its backward
// as batched gfx950 MFMA GEMMs.
//
// x (B, k p), w1 (k, q, p), w2 (l, s, r), k = l blocks, q = r:
//   forward   out1[kk][b][jq] = x[b][kk p : (kk+1) p] . w1[kk][jq]          (F1)
//             t[ll][b][i]     = out1 flat (b, i l + ll)   (the riffle)
//             out[b][ll][j]   = t[ll][b] . w2[ll][j]                         (F2)
//   backward  dw2[ll]  = dout[:, ll]^T t[ll]                                (B1)
//             dt[ll]   = dout[:, ll] w2[ll]                                 (B2)
//             dout1    = unriffle(dt);  dx[kk] = dout1[kk] w1[kk]           (B3)
//             dw1[kk]  = dout1[kk]^T x[kk]                                  (B4)
// (pretrain/src/models/monarch/monarch_ops.py:23-36, 57-82; the riffle and its
// inverse: monarch_riffle.py:13-57, 60-107.)
//
// The permutations cost no pass of their own: F1's epilogue writes t in riffled
// order (the staged tile is read back with the columns permuted), B3 reads dt
// with its K index permuted (K runs over (ll, j) and its w1 rows are j l + ll),
// B4 computes dw1 with its rows permuted and the split-K reduction writes them
// back in place.  bf16 operands, fp32 accumulation, bf16 results (the rounding
// points of the reference's bf16 bmms: out1, out, dt, dx, dw1, dw2).
//
// One GEMM kernel serves all six products: 256 x 256 output tiles per
// 512-thread workgroup, the MFMA pipeline and LDS slice forms of mfma_tile.hpp,
// operands K-major (K form) or MN-major (T form, read transposed with
// ds_read_b64_tr_b16), staged by buffer loads straight into LDS.  A buffer load
// whose lane offset is beyond the resource's range returns zeros, which pads
// partial tiles (token counts and block sides that are not multiples of 256)
// without branches in the loop.  The weight-gradient products contract over the
// tokens and have few output tiles; they split K and reduce the fp32 partials
// in a fixed order (deterministic).
#include <algorithm>
#include <atomic>

#include "common.hpp"
#include "kernels.hpp"
#include "mfma_tile.hpp"

namespace mmuon {
namespace {

typedef int i32x4 __attribute__((ext_vector_type(4)));

// Lane offset that reads zeros: the resource covers [0, OOB) bytes.
constexpr uint32_t OOB = 0x80000000u;

// Raw buffer resource over [base, base + OOB): base address, stride 0,
// num_records OOB, the gfx9 data-format word.
__device__ __forceinline__ i32x4 buffer_rsrc(const char* base) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  i32x4 r;
  r[0] = __builtin_amdgcn_readfirstlane(int(low_word(a)));
  r[1] = __builtin_amdgcn_readfirstlane(int(high_word(a) & 0xffffu));
  r[2] = int(OOB);
  r[3] = 0x00020000;
  return r;
}

// 16-B buffer load straight into LDS: lane l lands at lds + 16 l (M0 holds the
// wave-uniform LDS address).  Inline assembly for the same reason as dma16: the
// pipeline waits for exactly the slice it reads.
// m0 is listed as clobbered (the asm writes it); clang warns that m0 is a
// register it reserves for its own uses, which it sets right before each.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void bdma16(i32x4 rsrc, uint32_t voff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds"
               :
               : "v"(voff), "s"(rsrc), "s"(__builtin_amdgcn_readfirstlane(lds))
               : "memory", "m0");
}
#pragma clang diagnostic pop

// floor(n / d) for 0 <= n < 2^24, 1 <= d < 2^16, with magic = ceil(2^40 / d)
// (exact because n d < 2^40).
__host__ __device__ __forceinline__ int64_t seg_div(int64_t n, uint64_t magic) {
  return int64_t((uint64_t(n) * magic) >> 40);
}
uint64_t seg_magic(int64_t d) { return ((uint64_t(1) << 40) + uint64_t(d) - 1) / uint64_t(d); }

// GEMM operand: element (mn, k) of batch g sits at
//   base + g bstride + seg(mn) + seg(k),
//   seg(x) = (x / xseg) xseg_stride + (x % xseg) xstride.
// Segments express the riffle permutations; an unsegmented index has
// xseg > its extent.  K form: kstride == 2 (rows of K contiguous); T form:
// mstride == 2 (MN contiguous).  Indices mn >= extent read as zeros.
struct GOp {
  const char* base;
  int64_t bstride;
  int64_t mstride, mseg_stride;
  int64_t kstride, kseg_stride;
  uint64_t mmagic, kmagic;
  int32_t mseg, kseg;
  int32_t extent;
  int32_t pad;
};

__device__ __forceinline__ int64_t mn_off(const GOp& o, int64_t m) {
  const int64_t s = seg_div(m, o.mmagic);
  return s * o.mseg_stride + (m - s * o.mseg) * o.mstride;
}
// The K addressing of an operand, held by the main loop.
struct GOpK {
  int64_t kstride, kseg_stride;
  uint64_t kmagic;
  int64_t kseg;
};
__device__ __forceinline__ GOpK k_addr(const GOp& o) { return GOpK{o.kstride, o.kseg_stride, o.kmagic, o.kseg}; }
__device__ __forceinline__ int64_t k_off(const GOpK& o, int64_t k) {
  const int64_t s = seg_div(k, o.kmagic);
  return s * o.kseg_stride + (k - s * o.kseg) * o.kstride;
}

// bf16 result: row m of batch g at base + g bstride + seg(m), column n at
// 2 n; riffle (log2 l > 0): column jq of the tile's columns goes to plane
// jq % l, column jq / l (plane stride cplane).
struct GOut {
  char* base;
  int64_t bstride;
  int64_t rstride, rseg_stride;
  int64_t cplane;
  uint64_t rmagic;
  int32_t rseg;
  int32_t log2l;
};

struct GemmArgs {
  GOp a, b;        // row operand (M x K), column operand (N x K)
  GOut c;          // bf16 result (partial == null)
  float* partial;  // split-K: fp32 partials [S][G][M][N]
  int M, N, K, G, S;
  int kchunk;      // K per split, a multiple of BK
  int tiles_m, tiles_n;
  int vtiles;      // virtual tiles: 8 XCDs x ceil(G * S * tiles_m / 8) groups x tiles_n
};

// ---------------------------------------------------------------------------
// The pipelined main loop (the NS kernels' schedule with both operand forms
// fixed per launch): slice kt in ring slot kt % RING, RING - 2 slices in flight
// behind the one being read, fragment reads and buffer loads interleaved one
// per MFMA.  (A fifth slot, the whole LDS, measured slightly slower.)
// ---------------------------------------------------------------------------
constexpr int RING = 4;
constexpr int RING_ELEMS = RING * SLOT;
static_assert(RING_ELEMS * 2 <= 160 * 1024 && RING_ELEMS >= BN * 256, "ring and staged tile fit the LDS");
template <bool AT, bool BT>
struct GPipe {
  static_assert(RDMA == 2 && CDMA == 2, "two buffer loads per thread and operand slice");
  const char* abase;  // row operand at (tile row 0, k = 0) of this batch
  const char* bbase;
  GOpK ak, bk;        // K addressing of the two operands
  uint32_t loff[4];   // per-lane byte offsets of the four loads (OOB: beyond the extent)
  int kbeg, kend, KT;
  int wave, lane, wm, wn;
  uint16_t* lds;
  uint32_t lds0;
  uint32_t kfrag[BK / 16];
  uint32_t tfrag_r, tfrag_c;

  __device__ __forceinline__ const uint16_t* slot(int kt) const { return lds + (kt % RING) * SLOT; }

  // K delta of this lane's load q within a slice: K form, its 8-element chunk;
  // T form, its k row
  template <bool T>
  __device__ __forceinline__ int kdelta(int q) const {
    return T ? 16 * q + (lane >> 2) : 8 * ((lane & 3) ^ ((lane >> 4) & 3));
  }

  // Load Q (0, 1: row operand; 2, 3: column operand) of slice src_kt into the
  // slot of slice slot_kt.  K form: operand rows 16 (2w + q) + lane/4, chunk
  // (lane%4) ^ ((lane>>4)&3); T form: k rows 16 q + lane/4 of the slice,
  // MN 32 w + 8 (lane%4).  Either way the load lands at byte (2w + q) * 1024 of
  // the operand's slice.
  template <int Q>
  __device__ __forceinline__ void issue_one(int src_kt, int slot_kt) const {
    constexpr int q = Q & 1;
    constexpr bool T = Q < 2 ? AT : BT;
    const uint32_t dst = lds0 + (slot_kt % RING) * SLOT * 2 + (Q < 2 ? 0 : RSLICE * 2) + (2 * wave + q) * 1024;
    const int k0 = kbeg + src_kt * BK;
    const char* sb = (Q < 2 ? abase : bbase) + k_off(Q < 2 ? ak : bk, k0);
    uint32_t voff = loff[Q];
    const int rem = kend - k0;
    if (rem < BK && kdelta<T>(q) >= rem) voff = OOB;
    bdma16(buffer_rsrc(sb), voff, dst);
  }
  __device__ __forceinline__ void issue(int src_kt, int slot_kt) const {
    issue_one<0>(src_kt, slot_kt);
    issue_one<1>(src_kt, slot_kt);
    issue_one<2>(src_kt, slot_kt);
    issue_one<3>(src_kt, slot_kt);
  }

  template <int KK, int G>
  __device__ __forceinline__ void load_one(int kt, Frags& f) const {
    const uint16_t* sr = slot(kt);
    const uint16_t* sc = sr + RSLICE;
    if constexpr (G < TMJ)
      f.c[G] = BT ? frag_rowmajor_tr(sc, tfrag_c + G * 2048, KK) : frag_kmajor(sc, kfrag[KK], wn * WN + G * 32);
    else
      f.r[G - TMJ] = AT ? frag_rowmajor_tr(sr, tfrag_r + (G - TMJ) * 2048, KK)
                        : frag_kmajor(sr, kfrag[KK], wm * WM + (G - TMJ) * 32);
  }

  __device__ __forceinline__ void body(int kt, Frags& fa, Frags& fb, f32x16 (&acc)[TMI][TMJ]) const {
    static_assert(TMI * TMJ == 8 && SLICE_DMA <= 8 && TMI + TMJ <= 8, "one read / load per MFMA");
#define MMUON_GSTEP0(g)                                                                      \
    acc[(g) / TMJ][(g) % TMJ] = mfma(fa.r[(g) / TMJ], fa.c[(g) % TMJ], acc[(g) / TMJ][(g) % TMJ]); \
    if constexpr ((g) < TMI + TMJ) load_one<1, (g)>(kt, fb);                                 \
    __builtin_amdgcn_sched_barrier(0);
    MMUON_GSTEP0(0) MMUON_GSTEP0(1) MMUON_GSTEP0(2) MMUON_GSTEP0(3)
    MMUON_GSTEP0(4) MMUON_GSTEP0(5) MMUON_GSTEP0(6) MMUON_GSTEP0(7)
#undef MMUON_GSTEP0
    wait_vm<(RING - 3) * SLICE_DMA>();  // slice kt+1 landed
    barrier();
    const int src = kt + RING - 1 < KT ? kt + RING - 1 : KT - 1;
    const int slt = kt + RING - 1;
#define MMUON_GSTEP1(g)                                                                      \
    acc[(g) / TMJ][(g) % TMJ] = mfma(fb.r[(g) / TMJ], fb.c[(g) % TMJ], acc[(g) / TMJ][(g) % TMJ]); \
    if constexpr ((g) < TMI + TMJ) load_one<0, (g)>(kt + 1, fa);                             \
    if constexpr ((g) < SLICE_DMA) issue_one<(g)>(src, slt);                                 \
    __builtin_amdgcn_sched_barrier(0);
    // raised wave priority from the barrier to the end of k step 1, so the
    // SIMD's wave still in this phase wins issue over one already in the next
    // step and catches up before the next barrier
    __builtin_amdgcn_s_setprio(1);
    MMUON_GSTEP1(0) MMUON_GSTEP1(1) MMUON_GSTEP1(2) MMUON_GSTEP1(3)
    MMUON_GSTEP1(4) MMUON_GSTEP1(5) MMUON_GSTEP1(6) MMUON_GSTEP1(7)
#undef MMUON_GSTEP1
    __builtin_amdgcn_s_setprio(0);
  }

  __device__ __forceinline__ void run(f32x16 (&acc)[TMI][TMJ]) const {
#pragma unroll
    for (int i = 0; i < TMI; ++i)
#pragma unroll
      for (int j = 0; j < TMJ; ++j) acc[i][j] = f32x16{};
#pragma unroll
    for (int q = 0; q < RING - 1; ++q) issue(q < KT ? q : KT - 1, q);
    wait_vm<(RING - 2) * SLICE_DMA>();  // slice 0 landed
    barrier();
    Frags fa, fb;
    load_one<0, 0>(0, fa);
    load_one<0, 1>(0, fa);
    load_one<0, 2>(0, fa);
    load_one<0, 3>(0, fa);
    load_one<0, 4>(0, fa);
    load_one<0, 5>(0, fa);
    for (int kt = 0; kt < KT; ++kt) body(kt, fa, fb, acc);
    wait_vm<0>();  // the refills of the last steps land before the ring is reused
  }
};

// Per-lane byte offset of load q of an operand (tile origin mn0), OOB beyond
// its extent.
template <bool T>
__device__ __forceinline__ uint32_t lane_offset(const GOp& o, int mn0, int wave, int lane, int q) {
  int mn;
  int64_t off;
  if (T) {
    mn = mn0 + 32 * wave + 8 * (lane & 3);
    off = int64_t(16 * q + (lane >> 2)) * o.kstride;
  } else {
    mn = mn0 + 16 * (2 * wave + q) + (lane >> 2);
    off = int64_t((lane & 3) ^ ((lane >> 4) & 3)) * 16;
  }
  if (mn >= o.extent) return OOB;
  return uint32_t(off + mn_off(o, mn) - mn_off(o, mn0));
}

// Accumulators -> the staging area as T[j][i] = D[i][j] (tile_off layout), bf16.
__device__ __forceinline__ void stage_acc(char* stage, const f32x16 (&acc)[TMI][TMJ]) {
  const int tid = fresh_tid();
  const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / NWN, wn = wave % NWN;
#pragma unroll
  for (int i = 0; i < TMI; ++i)
#pragma unroll
    for (int j = 0; j < TMJ; ++j)
#pragma unroll
      for (int qg = 0; qg < 4; ++qg) {
        const f32x16& v = acc[i][j];
        const int row = wn * WN + j * 32 + (lane & 31);
        const int col = wm * WM + i * 32 + qg * 8 + (lane >> 5) * 4;
        *reinterpret_cast<uint2*>(stage + tile_off(row, col)) =
            make_uint2(f2bf2(v[qg * 4], v[qg * 4 + 1]), f2bf2(v[qg * 4 + 2], v[qg * 4 + 3]));
      }
}

// Staged tile -> destination rows.  Tile column order is permuted by the
// riffle: destination position dc (plane dc / (256/l), column dc % (256/l))
// holds tile column (dc % (256/l)) l + dc / (256/l).  ds_read_b64_tr_b16 on
// 16-lane groups: lanes 4e..4e+3 address staged row (tile column) R(e), four
// consecutive tile rows each, and lane i receives D[i0 + i][R(0..3)].  A wave
// task covers 16 tile rows x 64 destination columns; a lane writes two 16-B
// chunks.  fn(row, dc, uint4) stores destination columns dc .. dc+7 of a row.
template <class Fn>
__device__ __forceinline__ void write_tile(const char* stage, int log2l, Fn&& fn) {
  const int tid = fresh_tid();
  const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15, grp = lane >> 4;
  const int wshift = 8 - log2l, wmask = (1 << wshift) - 1;  // plane width 256 / l
  auto trow = [&](int dc) { return ((dc & wmask) << log2l) | (dc >> wshift); };
#pragma unroll 2
  for (int it = 0; it < 16 * 4 / NWAVES; ++it) {
    const int task = wave + NWAVES * it;
    const int i0 = (task & 15) * 16;
    const int tc = i0 + ((l16 & 3) << 2);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int dc = (task >> 4) * 64 + grp * 16 + h * 8;
      const i16x4 lo =
          __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(stage + tile_off(trow(dc + (l16 >> 2)), tc)));
      const i16x4 hi =
          __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(stage + tile_off(trow(dc + 4 + (l16 >> 2)), tc)));
      uint4 v;
      v.x = uint32_t(uint16_t(lo[0])) | (uint32_t(uint16_t(lo[1])) << 16);
      v.y = uint32_t(uint16_t(lo[2])) | (uint32_t(uint16_t(lo[3])) << 16);
      v.z = uint32_t(uint16_t(hi[0])) | (uint32_t(uint16_t(hi[1])) << 16);
      v.w = uint32_t(uint16_t(hi[2])) | (uint32_t(uint16_t(hi[3])) << 16);
      fn(i0 + l16, dc, v);
    }
  }
}

// Virtual tile v -> (batch g, split sp, tile row tm, tile column tn).  A group
// (g, sp, tm) is the tiles_n tiles that share a row-operand band; groups are
// numbered tm fastest and dealt to the XCDs in contiguous runs (virtual tile v
// runs on XCD v % 8), so the tiles of one XCD share one batch's column operand
// and few row bands, and each operand block is fetched from HBM by one or two
// XCDs rather than by all eight.
__device__ __forceinline__ bool decode_gemm_tile(const GemmArgs& a, int v, int& g, int& sp, int& tm, int& tn) {
  const int xcd = v & 7, local = v >> 3;
  const int ngroups = a.G * a.S * a.tiles_m;
  const int gpx = (ngroups + 7) / 8;  // groups per XCD
  const int lg = local / a.tiles_n;
  const int grp = xcd * gpx + lg;
  tn = local % a.tiles_n;
  if (lg >= gpx || grp >= ngroups) return false;
  tm = grp % a.tiles_m;
  sp = (grp / a.tiles_m) % a.S;
  g = grp / (a.tiles_m * a.S);
  return true;
}

template <bool AT, bool BT, bool SPLIT>
__device__ __forceinline__ void gemm_work(const GemmArgs& a, uint16_t* lds, int v) {
  int g, sp, tm, tn;
  if (!decode_gemm_tile(a, v, g, sp, tm, tn)) return;
  const int m0 = tm * BM, n0 = tn * BN;
  GPipe<AT, BT> p;
  p.lane = threadIdx.x & 63;
  p.wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  p.wm = p.wave / NWN;
  p.wn = p.wave % NWN;
  p.ak = k_addr(a.a);
  p.bk = k_addr(a.b);
  p.abase = a.a.base + int64_t(g) * a.a.bstride + mn_off(a.a, m0);
  p.bbase = a.b.base + int64_t(g) * a.b.bstride + mn_off(a.b, n0);
  p.kbeg = sp * a.kchunk;
  p.kend = min(a.K, p.kbeg + a.kchunk);
  p.KT = (p.kend - p.kbeg + BK - 1) / BK;
  p.loff[0] = lane_offset<AT>(a.a, m0, p.wave, p.lane, 0);
  p.loff[1] = lane_offset<AT>(a.a, m0, p.wave, p.lane, 1);
  p.loff[2] = lane_offset<BT>(a.b, n0, p.wave, p.lane, 0);
  p.loff[3] = lane_offset<BT>(a.b, n0, p.wave, p.lane, 1);
  p.lds = lds;
  p.lds0 = lds_addr(lds);
#pragma unroll
  for (int kk = 0; kk < BK / 16; ++kk) p.kfrag[kk] = kmajor_frag_base(kk, p.lane);
  p.tfrag_r = rowmajor_frag_base(p.wm * TMI, p.lane);
  p.tfrag_c = rowmajor_frag_base(p.wn * TMJ, p.lane);
  f32x16 acc[TMI][TMJ];
  p.run(acc);

  if constexpr (SPLIT) {
    // fp32 partial tile, straight from the accumulators: lane = one column,
    // 16 rows per MFMA tile; a wave store covers two 128-B row segments
    float* P = a.partial + (int64_t(sp) * a.G + g) * int64_t(a.M) * a.N;
    const int lane = p.lane;
#pragma unroll
    for (int i = 0; i < TMI; ++i)
#pragma unroll
      for (int j = 0; j < TMJ; ++j) {
        const int col = n0 + p.wn * WN + j * 32 + (lane & 31);
        if (col >= a.N) continue;
#pragma unroll
        for (int qg = 0; qg < 4; ++qg)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int row = m0 + p.wm * WM + i * 32 + qg * 8 + (lane >> 5) * 4 + e;
            if (row < a.M) P[int64_t(row) * a.N + col] = acc[i][j][qg * 4 + e];
          }
      }
  } else {
    char* stage = reinterpret_cast<char*>(lds);
    barrier();  // every wave is done with the ring
    stage_acc(stage, acc);
    barrier();
    const GOut& c = a.c;
    char* cb = c.base + int64_t(g) * c.bstride;
    const int wshift = 8 - c.log2l;
    const int ncol = (a.N - n0) >> c.log2l;  // valid destination columns per plane
    write_tile(stage, c.log2l, [&](int r, int dc, const uint4& u) {
      const int row = m0 + r;
      const int plane = dc >> wshift, col = dc & ((1 << wshift) - 1);
      if (row >= a.M || col >= ncol) return;
      const int64_t s = seg_div(row, c.rmagic);
      char* dst = cb + s * c.rseg_stride + (row - s * c.rseg) * c.rstride + plane * c.cplane +
                  int64_t((n0 >> c.log2l) + col) * 2;
      *reinterpret_cast<uint4*>(dst) = u;
    });
  }
}

template <bool AT, bool BT, bool SPLIT>
__global__ __launch_bounds__(NT, 1) void butterfly_gemm(GemmArgs a) {
  __shared__ __attribute__((aligned(1024))) uint16_t lds[RING_ELEMS];
  for (int v = blockIdx.x; v < a.vtiles; v += gridDim.x) {
    gemm_work<AT, BT, SPLIT>(a, lds, v);
    barrier();  // the staging area is read before the next tile's loads refill the ring
  }
}

// Split-K reduction: out row seg(m) of batch g, columns n..n+7 =
// bf16(sum over splits, in split order, of the fp32 partials).  S = 0 writes zeros.
__global__ __launch_bounds__(256) void splitk_reduce(const float* partial, int S, int G, int M, int N, GOut c) {
  const int n8 = N / 8;
  const int64_t total = int64_t(G) * M * n8;
  for (int64_t t = int64_t(blockIdx.x) * 256 + threadIdx.x; t < total; t += int64_t(gridDim.x) * 256) {
    const int n = int(t % n8) * 8;
    const int64_t gm = t / n8;
    const int m = int(gm % M), g = int(gm / M);
    float v[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int s = 0; s < S; ++s) {
      const float* p = partial + ((int64_t(s) * G + g) * M + m) * int64_t(N) + n;
      const float4 x = reinterpret_cast<const float4*>(p)[0];
      const float4 y = reinterpret_cast<const float4*>(p)[1];
      v[0] += x.x; v[1] += x.y; v[2] += x.z; v[3] += x.w;
      v[4] += y.x; v[5] += y.y; v[6] += y.z; v[7] += y.w;
    }
    const int64_t sg = seg_div(m, c.rmagic);
    uint16_t* dst = reinterpret_cast<uint16_t*>(c.base + int64_t(g) * c.bstride + sg * c.rseg_stride +
                                                (m - sg * c.rseg) * c.rstride) + n;
    uint4 r;
    r.x = f2bf2(v[0], v[1]);
    r.y = f2bf2(v[2], v[3]);
    r.z = f2bf2(v[4], v[5]);
    r.w = f2bf2(v[6], v[7]);
    *reinterpret_cast<uint4*>(dst) = r;
  }
}


// ---------------------------------------------------------------------------
// Host side: the six products as GemmArgs.
// ---------------------------------------------------------------------------
constexpr int64_t UNSEG = int64_t(1) << 24;  // segment length of an unsegmented index

GOp make_op(const void* base, int64_t bstride, int64_t mstride, int64_t kstride, int extent,
            int64_t mseg = UNSEG, int64_t mseg_stride = 0, int64_t kseg = UNSEG, int64_t kseg_stride = 0) {
  GOp o{};
  o.base = static_cast<const char*>(base);
  o.bstride = bstride;
  o.mstride = mstride;
  o.kstride = kstride;
  o.mseg = int32_t(mseg);
  o.mseg_stride = mseg_stride;
  o.kseg = int32_t(kseg);
  o.kseg_stride = kseg_stride;
  o.mmagic = seg_magic(mseg);
  o.kmagic = seg_magic(kseg);
  o.extent = extent;
  return o;
}

GOut make_out(void* base, int64_t bstride, int64_t rstride, int64_t rseg = UNSEG, int64_t rseg_stride = 0,
              int log2l = 0, int64_t cplane = 0) {
  GOut c{};
  c.base = static_cast<char*>(base);
  c.bstride = bstride;
  c.rstride = rstride;
  c.rseg = int32_t(rseg);
  c.rseg_stride = rseg_stride;
  c.rmagic = seg_magic(rseg);
  c.log2l = log2l;
  c.cplane = cplane;
  return c;
}

int cdiv(int64_t a, int64_t b) { return int((a + b - 1) / b); }

void set_geometry(GemmArgs& a, int M, int N, int K, int G, int S) {
  a.M = M;
  a.N = N;
  a.K = K;
  a.G = G;
  a.tiles_m = cdiv(M, BM);
  a.tiles_n = cdiv(N, BN);
  if (S > 1) {
    a.kchunk = cdiv(cdiv(K, S), BK) * BK;
    a.S = cdiv(K, a.kchunk);
  } else {
    a.kchunk = cdiv(std::max(K, 1), BK) * BK;
    a.S = 1;
  }
  a.vtiles = 8 * cdiv(int64_t(G) * a.S * a.tiles_m, 8) * a.tiles_n;
}

// Splits of a weight-gradient product (K = tokens), at least 1024 tokens per
// split: the S that minimises a cost model of a 256-CU part in units of one
// token of K per tile, rounds(S) (K/S + 576) + 768 [S > 1], where a round of
// tiles carries a fixed cost of about 576 (prologue, epilogue, store burst) and
// the fp32 partials' reduction pass about 768.  (6.89B at 4096 tokens: the
// 64-tile products split 4 ways, the 176-tile ones run unsplit, one round of
// K = 4096 instead of two of 2048 plus a reduction.)  A function of the shapes
// only, so the summation order (and the result) does not depend on the device.
int wgrad_splits(int M, int N, int G, int64_t K) {
  const int64_t tiles = int64_t(G) * cdiv(M, BM) * cdiv(N, BN);
  int best = 1;
  int64_t best_cost = -1;
  for (int S = 1; S <= 64 && (S == 1 || K >= int64_t(S) * 1024); S *= 2) {
    const int64_t rounds = (tiles * S + 255) / 256;
    const int64_t cost = rounds * ((K + S - 1) / S + 576) + (S > 1 ? 768 : 0);
    if (best_cost < 0 || cost < best_cost) {
      best = S;
      best_cost = cost;
    }
  }
  return best;
}

template <bool AT, bool BT, bool SPLIT>
void launch_gemm_t(const GemmArgs& a, hipStream_t s) {
  hipLaunchKernelGGL((butterfly_gemm<AT, BT, SPLIT>), dim3(resident_grid(a.vtiles)), dim3(NT), 0, s, a);
}

void launch_reduce(const GemmArgs& a, const GOut& c, hipStream_t s) {
  const int64_t total = int64_t(a.G) * a.M * (a.N / 8);
  const int blocks = int(std::min<int64_t>(std::max<int64_t>(1, (total + 255) / 256), 8192));
  hipLaunchKernelGGL(splitk_reduce, dim3(blocks), dim3(256), 0, s, a.partial, a.K > 0 ? a.S : 0, a.G, a.M, a.N, c);
}

struct Dims {
  int64_t B;
  int nb, q, p, s, log2l;
};

Dims dims(const mmuon_butterfly_args& x) {
  Dims d{x.tokens, x.nblocks, x.q, x.p, x.s, 0};
  while ((1 << d.log2l) < d.nb) ++d.log2l;
  return d;
}

}  // namespace

size_t butterfly_workspace(const mmuon_butterfly_args& x) {
  const Dims d = dims(x);
  const size_t dt = size_t(d.nb) * d.B * d.q * 2;
  const int s1 = wgrad_splits(d.s, d.q, d.nb, d.B), s4 = wgrad_splits(d.q, d.p, d.nb, d.B);
  const size_t part = std::max(size_t(s1) * d.nb * d.s * d.q, size_t(s4) * d.nb * d.q * d.p) * 4;
  return (dt + 255) / 256 * 256 + part;
}

int launch_butterfly_fwd(const mmuon_butterfly_args& x, hipStream_t st) {
  const Dims d = dims(x);
  if (d.B == 0) return 0;
  const int64_t n = int64_t(d.nb) * d.p, ql = d.q / d.nb;
  GemmArgs f1{};  // out1 (riffled into t) = x . w1^T per block kk
  f1.a = make_op(x.x, d.p * 2, n * 2, 2, int(d.B));
  f1.b = make_op(x.w1, int64_t(d.q) * d.p * 2, int64_t(d.p) * 2, 2, d.q);
  f1.c = make_out(x.out1, ql * 2, int64_t(d.q) * 2, UNSEG, 0, d.log2l, d.B * d.q * 2);
  set_geometry(f1, int(d.B), d.q, d.p, d.nb, 1);
  launch_gemm_t<false, false, false>(f1, st);
  GemmArgs f2{};  // out[:, ll] = t[ll] . w2[ll]^T
  f2.a = make_op(x.out1, d.B * d.q * 2, int64_t(d.q) * 2, 2, int(d.B));
  f2.b = make_op(x.w2, int64_t(d.s) * d.q * 2, int64_t(d.q) * 2, 2, d.s);
  f2.c = make_out(x.out, int64_t(d.s) * 2, int64_t(d.nb) * d.s * 2);
  set_geometry(f2, int(d.B), d.s, d.q, d.nb, 1);
  launch_gemm_t<false, false, false>(f2, st);
  return 0;
}

int launch_butterfly_bwd(const mmuon_butterfly_args& x, hipStream_t st) {
  const Dims d = dims(x);
  const int64_t n = int64_t(d.nb) * d.p, ql = d.q / d.nb;
  char* ws = static_cast<char*>(x.workspace);
  void* dt = ws;
  float* part = reinterpret_cast<float*>(ws + (size_t(d.nb) * d.B * d.q * 2 + 255) / 256 * 256);

  // dw2[ll] = dout[:, ll]^T t[ll]  (K = tokens, split; unsplit: bf16 straight
  // from the tile)
  GemmArgs b1{};
  b1.a = make_op(x.dout, int64_t(d.s) * 2, 2, int64_t(d.nb) * d.s * 2, d.s);
  b1.b = make_op(x.out1, d.B * d.q * 2, 2, int64_t(d.q) * 2, d.q);
  b1.partial = part;
  b1.c = make_out(x.dw2, int64_t(d.s) * d.q * 2, int64_t(d.q) * 2);
  set_geometry(b1, d.s, d.q, int(d.B), d.nb, wgrad_splits(d.s, d.q, d.nb, d.B));
  if (d.B > 0 && b1.S == 1) {
    launch_gemm_t<true, true, false>(b1, st);
  } else {
    if (d.B > 0) launch_gemm_t<true, true, true>(b1, st);
    launch_reduce(b1, b1.c, st);
  }
  if (d.B == 0) {
    GemmArgs b4{};
    b4.partial = part;
    set_geometry(b4, d.q, d.p, 0, d.nb, 1);
    launch_reduce(b4, make_out(x.dw1, int64_t(d.q) * d.p * 2, int64_t(d.p) * 2), st);
    return 0;
  }

  GemmArgs b2{};  // dt[ll] = dout[:, ll] w2[ll]
  b2.a = make_op(x.dout, int64_t(d.s) * 2, int64_t(d.nb) * d.s * 2, 2, int(d.B));
  b2.b = make_op(x.w2, int64_t(d.s) * d.q * 2, 2, int64_t(d.q) * 2, d.q);
  b2.c = make_out(dt, d.B * d.q * 2, int64_t(d.q) * 2);
  set_geometry(b2, int(d.B), d.q, d.s, d.nb, 1);
  launch_gemm_t<false, true, false>(b2, st);

  // dx[:, kk] = sum over (ll, j) of dt[ll][:, kk q/l + j] w1[kk][j l + ll]: K in
  // segments of q/l, one per plane ll (the unriffle folded into the addressing)
  GemmArgs b3{};
  b3.a = make_op(dt, ql * 2, int64_t(d.q) * 2, 2, int(d.B), UNSEG, 0, ql, d.B * d.q * 2);
  b3.b = make_op(x.w1, int64_t(d.q) * d.p * 2, 2, int64_t(d.nb) * d.p * 2, d.p, UNSEG, 0, ql, int64_t(d.p) * 2);
  b3.c = make_out(x.dx, int64_t(d.p) * 2, n * 2);
  set_geometry(b3, int(d.B), d.p, d.q, d.nb, 1);
  launch_gemm_t<false, true, false>(b3, st);

  // dw1[kk] with rows in (ll, j) order: row ll q/l + j of the product is
  // dw1 row j l + ll (the reduction writes it there)
  GemmArgs b4{};
  b4.a = make_op(dt, ql * 2, 2, int64_t(d.q) * 2, d.q, ql, d.B * d.q * 2);
  b4.b = make_op(x.x, int64_t(d.p) * 2, 2, n * 2, d.p);
  b4.partial = part;
  b4.c = make_out(x.dw1, int64_t(d.q) * d.p * 2, int64_t(d.nb) * d.p * 2, ql, int64_t(d.p) * 2);
  set_geometry(b4, d.q, d.p, int(d.B), d.nb, wgrad_splits(d.q, d.p, d.nb, d.B));
  if (b4.S == 1) {
    launch_gemm_t<true, true, false>(b4, st);
  } else {
    launch_gemm_t<true, true, true>(b4, st);
    launch_reduce(b4, b4.c, st);
  }
  return 0;
}

}  // namespace mmuon
