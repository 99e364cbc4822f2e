// extern "C" entry points of libmmuon.so (declared in include/mmuon.h).
// Argument validation, workspace geometry, stage sequencing; every launch on
// the caller's stream, no synchronisation, no device allocation.
#include <stdarg.h>
#include <stdio.h>

#include <algorithm>
#include <cmath>
#include <string>
#include <vector>

#include "common.hpp"
#include "kernels.hpp"

namespace mmuon {
int fp8_pack_nparts(int rows, int cols, bool transposed);
}

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(MMUON_EHIP, "%s: %s", what, hipGetErrorString(e));
  return MMUON_OK;
}

int64_t roundup(int64_t x, int64_t m) { return (x + m - 1) / m * m; }

int dtype_size(int dt) {
  switch (dt) {
    case MMUON_F32: return 4;
    case MMUON_BF16: return 2;
    case MMUON_F8E4M3: return 1;
    case MMUON_F8E5M2: return 1;
  }
  return 0;
}

bool is_fp8(int dt) { return dt == MMUON_F8E4M3 || dt == MMUON_F8E5M2; }

// expand_min of the FP8 codec: a positive finite number
int check_expand_min(float e) {
  if (!(e > 0.f) || !(e <= 3.4e38f)) return fail(MMUON_EINVAL, "expand_min must be positive and finite (got %g)", e);
  return MMUON_OK;
}

struct Geometry {
  int m, n, mp, np_, nparts;
  bool transposed;
};

int geometry(int rows, int cols, int ns_dtype, Geometry& g) {
  if (rows <= 0 || cols <= 0) return fail(MMUON_EINVAL, "block shape must be positive (%d x %d)", rows, cols);
  if (ns_dtype != MMUON_BF16 && ns_dtype != MMUON_F32)
    return fail(MMUON_EINVAL, "ns_dtype must be MMUON_BF16 or MMUON_F32 (got %d)", ns_dtype);
  g.transposed = rows > cols;
  g.m = std::min(rows, cols);
  g.n = std::max(rows, cols);
  const int tm = mmuon::ns_tile_m(ns_dtype), tn = mmuon::ns_tile_n(ns_dtype);
  const int64_t mp = roundup(g.m, tm), np_ = roundup(g.n, std::max(tn, 64));
  if (mp > (1 << 15) || np_ > (1 << 15)) return fail(MMUON_ERANGE, "block side beyond 32768 (%d x %d)", rows, cols);
  g.mp = int(mp);
  g.np_ = int(np_);
  g.nparts = std::max(mmuon::pack_nparts(g.mp, g.np_, g.transposed),
                      (int64_t(rows) * cols) % 128 == 0 ? mmuon::fp8_pack_nparts(rows, cols, g.transposed) : 0);
  return MMUON_OK;
}

int check_group(const mmuon_group* g, Geometry& geo) {
  if (g == nullptr) return fail(MMUON_EINVAL, "null group");
  if (g->nblocks <= 0) return fail(MMUON_EINVAL, "nblocks must be positive");
  if (g->blocks == nullptr) return fail(MMUON_EINVAL, "null block table");
  if (g->param_dtype != MMUON_F32 && g->param_dtype != MMUON_BF16)
    return fail(MMUON_EINVAL, "param dtype must be F32 or BF16");
  if (g->grad_dtype != MMUON_F32 && g->grad_dtype != MMUON_BF16)
    return fail(MMUON_EINVAL, "grad dtype must be F32 or BF16");
  if (int rc = geometry(g->rows, g->cols, g->ns_dtype, geo)) return rc;
  if (g->x0 == nullptr || g->x1 == nullptr || g->a == nullptr || g->p == nullptr ||
      g->partial == nullptr || g->scale == nullptr)
    return fail(MMUON_EINVAL, "workspace pointer missing");
  if ((reinterpret_cast<uintptr_t>(g->x0) | reinterpret_cast<uintptr_t>(g->x1) |
       reinterpret_cast<uintptr_t>(g->a) | reinterpret_cast<uintptr_t>(g->p)) & 15u)
    return fail(MMUON_EINVAL, "workspace stacks must be 16-byte aligned");
  return MMUON_OK;
}

mmuon::PackArgs pack_args(const mmuon_group* g, const Geometry& geo, float mu, int nparts) {
  mmuon::PackArgs a{};
  a.blocks = g->blocks;
  a.x = g->x0;
  a.partial = g->partial;
  a.N = g->nblocks;
  a.m = geo.m;
  a.n = geo.n;
  a.mp = geo.mp;
  a.np = geo.np_;
  a.nparts = nparts;
  a.mu = mu;
  a.gscale = g->grad_scale;
  return a;
}

}  // namespace

namespace mmuon {

int set_error(int code, const char* msg) { return fail(code, "%s", msg); }

int launch_status(const char* what) { return check_launch(what); }

int check_grad_norm_args(const mmuon_grad_norm_args* a, bool workspace) {
  if (a == nullptr) return fail(MMUON_EINVAL, "null gradient-norm arguments");
  if (a->grad_dtype != MMUON_F32 && a->grad_dtype != MMUON_BF16)
    return fail(MMUON_EINVAL, "gradient dtype must be F32 or BF16");
  if (a->nchunks < 0 || a->ntensors < 0) return fail(MMUON_EINVAL, "negative chunk or tensor count");
  if (a->nchunks > 0x7fffffff) return fail(MMUON_ERANGE, "too many gradient chunks");
  if (a->chunk_elems <= 0) return fail(MMUON_EINVAL, "chunk_elems must be positive");
  if (!a->total || !a->coef || (a->nchunks > 0 && (!a->tensors || !a->chunks)) || !a->first_chunk)
    return fail(MMUON_EINVAL, "null gradient-norm pointer");
  if (workspace && (!a->norms || (a->nchunks > 0 && !a->partial)))
    return fail(MMUON_EINVAL, "null gradient-norm workspace pointer");
  return MMUON_OK;
}

}  // namespace mmuon

extern "C" {

const char* mmuon_last_error(void) { return g_err.c_str(); }

int mmuon_abi_version(void) { return 7; }

int mmuon_ns_layout(int32_t rows, int32_t cols, int32_t ns_dtype, int64_t nblocks,
                    mmuon_ns_layout_t* out) {
  if (out == nullptr) return fail(MMUON_EINVAL, "null layout output");
  if (nblocks <= 0) return fail(MMUON_EINVAL, "nblocks must be positive");
  Geometry geo;
  if (int rc = geometry(rows, cols, ns_dtype, geo)) return rc;
  const int es = dtype_size(ns_dtype);
  out->m = geo.m;
  out->n = geo.n;
  out->mp = geo.mp;
  out->np_ = geo.np_;
  out->nparts = geo.nparts;
  out->ns_dtype = ns_dtype;
  out->x_bytes = nblocks * int64_t(geo.mp) * geo.np_ * es;
  out->a_bytes = nblocks * int64_t(geo.mp) * geo.mp * es;
  out->part_bytes = nblocks * int64_t(geo.nparts) * 4;
  return MMUON_OK;
}

int mmuon_momentum_pack(const mmuon_group* g, float momentum, void* stream) {
  Geometry geo;
  if (int rc = check_group(g, geo)) return rc;
  if (g->buf_dtype != MMUON_F32 && g->buf_dtype != MMUON_BF16)
    return fail(MMUON_EINVAL, "momentum dtype must be F32 or BF16 (FP8 uses mmuon_fp8_momentum_pack)");
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const int nparts = mmuon::pack_nparts(geo.mp, geo.np_, geo.transposed);
  mmuon::PackArgs a = pack_args(g, geo, momentum, nparts);
  const int row_len = geo.transposed ? geo.m : geo.n;  // length of a stored block row
  a.vec = ((g->flags & MMUON_GROUP_ALIGNED16) && row_len % 8 == 0) ? 1 : 0;
  if (mmuon::launch_pack(a, g->grad_dtype, g->buf_dtype, g->ns_dtype, geo.transposed, s))
    return fail(MMUON_EINVAL, "unsupported dtype combination grad=%d buf=%d ns=%d", g->grad_dtype,
                g->buf_dtype, g->ns_dtype);
  mmuon::launch_block_scale(g->partial, nparts, g->scale, g->nblocks, g->ns_dtype == MMUON_BF16, s);
  return check_launch("mmuon_momentum_pack");
}

int mmuon_fp8_momentum_pack(const mmuon_group* g, float momentum, int32_t have_state, float expand_min,
                            void* stream) {
  Geometry geo;
  if (int rc = check_group(g, geo)) return rc;
  if (!is_fp8(g->buf_dtype)) return fail(MMUON_EINVAL, "buf dtype must be MMUON_F8E4M3 or MMUON_F8E5M2");
  if (int rc = check_expand_min(expand_min)) return rc;
  if (g->fp8 == nullptr) return fail(MMUON_EINVAL, "null FP8 metadata table");
  if ((int64_t(g->rows) * g->cols) % 128 != 0)
    return fail(MMUON_EINVAL, "FP8 momentum needs rows*cols %% 128 == 0 (got %d x %d)", g->rows, g->cols);
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const int nparts = mmuon::fp8_pack_nparts(g->rows, g->cols, geo.transposed);
  mmuon::PackArgs a = pack_args(g, geo, momentum, nparts);
  if (mmuon::launch_fp8_pack(a, g->fp8, g->rows, g->cols, g->grad_dtype, g->ns_dtype, g->buf_dtype,
                             geo.transposed, have_state ? 1 : 0, expand_min, s))
    return fail(MMUON_EINVAL, "unsupported dtype combination grad=%d ns=%d", g->grad_dtype, g->ns_dtype);
  mmuon::launch_block_scale(g->partial, nparts, g->scale, g->nblocks, g->ns_dtype == MMUON_BF16, s);
  return check_launch("mmuon_fp8_momentum_pack");
}

}  // extern "C"

namespace {

// ---------------------------------------------------------------------------
// Newton-Schulz plans.  A plan is the list of stage launches of one group's
// iterations; mmuon_newton_schulz_apply runs it, mmuon_ns_plan hands it to the
// caller (per-launch timing, the stage tests) and mmuon_ns_run_op runs one op.
//
// Standard chain, per iteration: A = X X^T; P = a I + b A + c A A; X = P X
// (the a X term on P's diagonal).  Gram form (bf16 groups with n >= 2m after
// padding, 5 iterations): every X_k = Q_k X_0 with Q_k a polynomial in the
// first Gram matrix A_0, so the iterations can run on m x m matrices:
//   P_k = a I + b A_k + c A_k^2,  Q_{k+1} = P_k Q_k,  A_{k+1} = P_k (P_k A_k)
// (all symmetric and commuting: products of polynomials in A_0).  This
// replaces the two m x m x n products of an iteration by m x m x m ones.  In
// bf16 the Gram recursion alone drifts on ill-conditioned blocks, so X is
// rebuilt once, X_3 = Q_3 X_0, and the last two iterations restart from A_3 =
// X_3 X_3^T (three Gram iterations, restart, two).  The m x m intermediates
// beyond A and P use the idle X stack's memory (n >= 2m: two m x m stacks fit
// in one m x n stack).
// ---------------------------------------------------------------------------
bool is_x(int b) { return b == MMUON_NSB_X0 || b == MMUON_NSB_X1; }
bool is_sym(int b) {
  return b == MMUON_NSB_A || b == MMUON_NSB_P || (b >= MMUON_NSB_X0_S0 && b <= MMUON_NSB_X1_S1);
}
// the X stack whose memory holds sub-stack b (or b itself), -1 for A, P
int x_home(int b) {
  if (b == MMUON_NSB_X0 || b == MMUON_NSB_X0_S0 || b == MMUON_NSB_X0_S1) return MMUON_NSB_X0;
  if (b == MMUON_NSB_X1 || b == MMUON_NSB_X1_S0 || b == MMUON_NSB_X1_S1) return MMUON_NSB_X1;
  return -1;
}
bool overlaps(int u, int v) {
  if (u == v) return true;
  const int hu = x_home(u), hv = x_home(v);
  // a sub-stack overlaps its X stack; the two sub-stacks of one X stack do not
  return hu >= 0 && hu == hv && (is_x(u) || is_x(v));
}

bool gram_eligible(const Geometry& geo, int ns_dtype, int iters, int flags) {
  return ns_dtype == MMUON_BF16 && !(flags & MMUON_NS_STANDARD) && iters == 5 &&
         int64_t(geo.np_) >= 2 * int64_t(geo.mp);
}

void build_plan(const Geometry& geo, int ns_dtype, int iters, int flags, std::vector<mmuon_ns_op>& ops) {
  ops.clear();
  const bool apply = !(flags & MMUON_NS_NO_APPLY);
  auto op = [&](int kind, int in0, int in1, int out, int scaled, int it) {
    ops.push_back(mmuon_ns_op{kind, in0, in1, out, scaled, it});
  };
  if (!gram_eligible(geo, ns_dtype, iters, flags)) {
    for (int it = 0; it < iters; ++it) {
      const int cur = (it & 1) ? MMUON_NSB_X1 : MMUON_NSB_X0;
      const int nxt = (it & 1) ? MMUON_NSB_X0 : MMUON_NSB_X1;
      op(MMUON_NSOP_SYRK, cur, -1, MMUON_NSB_A, it == 0, it);
      op(MMUON_NSOP_POLY, MMUON_NSB_A, -1, MMUON_NSB_P, 0, it);
      if (apply && it + 1 == iters) op(MMUON_NSOP_PX_APPLY, MMUON_NSB_P, cur, MMUON_NSB_PARAM, it == 0, it);
      else op(MMUON_NSOP_PX, MMUON_NSB_P, cur, nxt, it == 0, it);
    }
    return;
  }
  enum { X0 = MMUON_NSB_X0, X1 = MMUON_NSB_X1, A = MMUON_NSB_A, P = MMUON_NSB_P,
         X0S0 = MMUON_NSB_X0_S0, X1S0 = MMUON_NSB_X1_S0, X1S1 = MMUON_NSB_X1_S1 };
  const int SYRK = MMUON_NSOP_SYRK, POLY = MMUON_NSOP_POLY, SYMM = MMUON_NSOP_SYMM;
  // iteration 0 (X_0 in x0, scaled by s): A_0, P_0 = Q_1, A_1 = P_0 (P_0 A_0)
  op(SYRK, X0, -1, A, 1, 0);
  op(POLY, A, -1, P, 0, 0);
  op(SYMM, P, A, X1S0, 0, 0);
  op(SYMM, P, X1S0, A, 0, 0);
  // iteration 1: P_1, Q_2 = P_1 Q_1, A_2 = P_1 (P_1 A_1)
  op(POLY, A, -1, X1S0, 0, 1);
  op(SYMM, X1S0, P, X1S1, 0, 1);
  op(SYMM, X1S0, A, P, 0, 1);
  op(SYMM, X1S0, P, A, 0, 1);
  // iteration 2: P_2, Q_3 = P_2 Q_2, restart X_3 = s Q_3 X_0 (into x1)
  op(POLY, A, -1, P, 0, 2);
  op(SYMM, P, X1S1, A, 0, 2);
  op(MMUON_NSOP_PX, A, X0, X1, 1, 2);
  // iteration 3: A_3 = X_3 X_3^T, P_3 = Q_4, A_4 = P_3 (P_3 A_3)
  op(SYRK, X1, -1, A, 0, 3);
  op(POLY, A, -1, P, 0, 3);
  op(SYMM, P, A, X0S0, 0, 3);
  op(SYMM, P, X0S0, A, 0, 3);
  // iteration 4: P_4, Q_5 = P_4 Q_4, X_5 = Q_5 X_3 (applied, or into x0)
  op(POLY, A, -1, X0S0, 0, 4);
  op(SYMM, X0S0, P, A, 0, 4);
  if (apply) op(MMUON_NSOP_PX_APPLY, A, X1, MMUON_NSB_PARAM, 0, 4);
  else op(MMUON_NSOP_PX, A, X1, X0, 0, 4);
}

int check_op(const Geometry& geo, int ns_dtype, const mmuon_ns_op* op) {
  if (op == nullptr) return fail(MMUON_EINVAL, "null Newton-Schulz op");
  const int k = op->kind, i0 = op->in0, i1 = op->in1, o = op->out;
  bool ok;
  switch (k) {
    case MMUON_NSOP_SYRK: ok = is_x(i0) && is_sym(o); break;
    case MMUON_NSOP_POLY: ok = is_sym(i0) && is_sym(o); break;
    case MMUON_NSOP_SYMM: ok = is_sym(i0) && is_sym(i1) && is_sym(o); break;
    case MMUON_NSOP_PX: ok = is_sym(i0) && is_x(i1) && is_x(o); break;
    case MMUON_NSOP_PX_APPLY: ok = is_sym(i0) && is_x(i1) && o == MMUON_NSB_PARAM; break;
    default: return fail(MMUON_EINVAL, "unknown Newton-Schulz op kind %d", k);
  }
  if (!ok) return fail(MMUON_EINVAL, "op kind %d: operand or output buffer of the wrong kind (%d, %d -> %d)", k, i0,
                       i1, o);
  const bool two = k == MMUON_NSOP_SYMM || k == MMUON_NSOP_PX || k == MMUON_NSOP_PX_APPLY;
  if (overlaps(o, i0) || (two && overlaps(o, i1)))
    return fail(MMUON_EINVAL, "op kind %d: output %d overlaps an operand", k, o);
  for (int b : {i0, two ? i1 : i0, o})
    if (b >= MMUON_NSB_X0_S0 && b <= MMUON_NSB_X1_S1 && int64_t(geo.np_) < 2 * int64_t(geo.mp))
      return fail(MMUON_EINVAL, "sub-stacks of an X stack need np >= 2 mp (mp %d, np %d)", geo.mp, geo.np_);
  if (k == MMUON_NSOP_SYMM && ns_dtype != MMUON_BF16)
    return fail(MMUON_EINVAL, "the symmetric product runs on bf16 groups only");
  return MMUON_OK;
}

void* buf_ptr(const mmuon_group* g, const Geometry& geo, int b) {
  const int64_t sub = int64_t(g->nblocks) * geo.mp * geo.mp * dtype_size(g->ns_dtype);
  char* x0 = static_cast<char*>(g->x0);
  char* x1 = static_cast<char*>(g->x1);
  switch (b) {
    case MMUON_NSB_X0: case MMUON_NSB_X0_S0: return x0;
    case MMUON_NSB_X1: case MMUON_NSB_X1_S0: return x1;
    case MMUON_NSB_X0_S1: return x0 + sub;
    case MMUON_NSB_X1_S1: return x1 + sub;
    case MMUON_NSB_A: return g->a;
    case MMUON_NSB_P: return g->p;
  }
  return nullptr;
}

int run_op(const mmuon_group* g, const Geometry& geo, const mmuon_ns_op& op, const float coeffs[3], float alpha,
           hipStream_t s) {
  if (int rc = check_op(geo, g->ns_dtype, &op)) return rc;
  mmuon::NsArgs a{};
  a.blocks = g->blocks;
  a.N = g->nblocks;
  a.m = geo.m;
  a.n = geo.n;
  a.mp = geo.mp;
  a.np = geo.np_;
  a.kx = int(roundup(geo.n, mmuon::ns_tile_k(g->ns_dtype)));
  a.ca = coeffs[0];
  a.cb = coeffs[1];
  a.cc = coeffs[2];
  a.alpha = alpha;
  a.transposed = geo.transposed ? 1 : 0;
  a.vec = (g->flags & MMUON_GROUP_ALIGNED16) ? 1 : 0;
  const float* sc = op.scaled ? g->scale : nullptr;
  int kstage = 0;
  switch (op.kind) {
    case MMUON_NSOP_SYRK:
      a.scale = sc;
      a.x_in = buf_ptr(g, geo, op.in0);
      kstage = mmuon::NS_SYRK;
      break;
    case MMUON_NSOP_POLY:
      a.a_in = buf_ptr(g, geo, op.in0);
      kstage = mmuon::NS_POLY;
      break;
    case MMUON_NSOP_SYMM:
      a.a_in = buf_ptr(g, geo, op.in0);
      a.b_in = buf_ptr(g, geo, op.in1);
      kstage = mmuon::NS_SYMM;
      break;
    default:  // PX, PX_APPLY
      a.scale = sc;
      a.a_in = buf_ptr(g, geo, op.in0);
      a.x_in = buf_ptr(g, geo, op.in1);
      kstage = op.kind == MMUON_NSOP_PX ? mmuon::NS_PX : mmuon::NS_PX_APPLY;
      break;
  }
  a.out = op.out == MMUON_NSB_PARAM ? nullptr : buf_ptr(g, geo, op.out);
  if (mmuon::launch_ns_stage(a, kstage, g->ns_dtype, g->param_dtype, s))
    return fail(MMUON_EINVAL, "no Newton-Schulz kernel for op %d, ns dtype %d / param dtype %d", op.kind,
                g->ns_dtype, g->param_dtype);
  return MMUON_OK;
}

int check_ns(const mmuon_group* g, Geometry& geo, int iters, const float* coeffs) {
  if (int rc = check_group(g, geo)) return rc;
  if (iters < 1 || iters > 64) return fail(MMUON_EINVAL, "iters must be in [1, 64] (got %d)", iters);
  if (coeffs == nullptr) return fail(MMUON_EINVAL, "null coefficients");
  return MMUON_OK;
}

}  // namespace

extern "C" {

int mmuon_ns_plan(int32_t rows, int32_t cols, int32_t ns_dtype, int32_t iters, int32_t flags, mmuon_ns_op* ops,
                  int32_t max_ops) {
  Geometry geo;
  if (int rc = geometry(rows, cols, ns_dtype, geo)) return rc;
  if (iters < 1 || iters > 64) return fail(MMUON_EINVAL, "iters must be in [1, 64] (got %d)", iters);
  std::vector<mmuon_ns_op> plan;
  build_plan(geo, ns_dtype, iters, flags, plan);
  const int n = int(plan.size());
  if (ops != nullptr) {
    if (max_ops < n) return fail(MMUON_ERANGE, "plan has %d ops, room for %d", n, max_ops);
    std::copy(plan.begin(), plan.end(), ops);
  }
  return n;
}

int mmuon_ns_run_op(const mmuon_group* g, const mmuon_ns_op* op, const float coeffs[3], float alpha,
                    void* stream) {
  Geometry geo;
  if (int rc = check_ns(g, geo, 1, coeffs)) return rc;
  if (op == nullptr) return fail(MMUON_EINVAL, "null Newton-Schulz op");
  if (int rc = run_op(g, geo, *op, coeffs, alpha, static_cast<hipStream_t>(stream))) return rc;
  return check_launch("mmuon_ns_run_op");
}

int mmuon_newton_schulz_apply(const mmuon_group* g, int32_t iters, const float coeffs[3], float alpha,
                              int32_t flags, void* stream) {
  Geometry geo;
  if (int rc = check_ns(g, geo, iters, coeffs)) return rc;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  std::vector<mmuon_ns_op> plan;
  build_plan(geo, g->ns_dtype, iters, flags, plan);
  const size_t nrun = (flags & MMUON_NS_HOLD_LAST) ? plan.size() - 1 : plan.size();
  for (size_t i = 0; i < nrun; ++i)
    if (int rc = run_op(g, geo, plan[i], coeffs, alpha, s)) return rc;
  return check_launch("mmuon_newton_schulz_apply");
}

int mmuon_ns_stage(const mmuon_group* g, int32_t iteration, int32_t iters, int32_t stage,
                   const float coeffs[3], float alpha, int32_t flags, void* stream) {
  Geometry geo;
  if (int rc = check_ns(g, geo, iters, coeffs)) return rc;
  if (iteration < 0 || iteration >= iters)
    return fail(MMUON_EINVAL, "iteration %d outside [0, %d)", iteration, iters);
  if (stage < 0 || stage > 2) return fail(MMUON_EINVAL, "stage must be 0, 1 or 2 (got %d)", stage);
  std::vector<mmuon_ns_op> plan;
  build_plan(geo, g->ns_dtype, iters, flags | MMUON_NS_STANDARD, plan);
  if (int rc = run_op(g, geo, plan[size_t(3 * iteration + stage)], coeffs, alpha, static_cast<hipStream_t>(stream)))
    return rc;
  return check_launch("mmuon_ns_stage");
}

namespace {
int check_adamw(const mmuon_adamw_args* a) {
  if (a == nullptr) return fail(MMUON_EINVAL, "null AdamW arguments");
  if (a->nchunks < 0) return fail(MMUON_EINVAL, "negative chunk count");
  if (a->nchunks > 0 && (a->tensors == nullptr || a->chunks == nullptr))
    return fail(MMUON_EINVAL, "null AdamW tables");
  if (a->nchunks > 0x7fffffff) return fail(MMUON_ERANGE, "too many AdamW chunks");
  if (a->chunk_elems <= 0) return fail(MMUON_EINVAL, "chunk_elems must be positive");
  return MMUON_OK;
}
mmuon::AdamWArgs adamw_args(const mmuon_adamw_args* a) {
  mmuon::AdamWArgs k{};
  k.tensors = a->tensors;
  k.chunks = a->chunks;
  k.nchunks = a->nchunks;
  k.chunk_elems = a->chunk_elems;
  k.wd_factor = a->wd_factor;
  k.apply_wd = a->apply_weight_decay ? 1 : 0;
  k.beta1 = a->beta1;
  k.one_minus_beta1 = a->one_minus_beta1;
  k.beta2 = a->beta2;
  k.one_minus_beta2 = a->one_minus_beta2;
  k.sqrt_bc2 = a->sqrt_bc2;
  k.eps = a->eps;
  k.neg_step_size = a->neg_step_size;
  k.gscale = a->grad_scale;
  return k;
}
}  // namespace

int mmuon_adamw(const mmuon_adamw_args* a, void* stream) {
  if (int rc = check_adamw(a)) return rc;
  const mmuon::AdamWArgs k = adamw_args(a);
  if (mmuon::launch_adamw(k, a->param_dtype, a->grad_dtype, a->state_dtype, static_cast<hipStream_t>(stream)))
    return fail(MMUON_EINVAL, "unsupported AdamW dtypes param=%d grad=%d state=%d", a->param_dtype,
                a->grad_dtype, a->state_dtype);
  return check_launch("mmuon_adamw");
}

int mmuon_adamw_fp8(const mmuon_adamw_args* a, const mmuon_adamw_fp8_tensor* meta, int32_t have_state,
                    int32_t v_dtype, float expand_min, void* stream) {
  if (int rc = check_adamw(a)) return rc;
  if (a->chunk_elems != 128) return fail(MMUON_EINVAL, "FP8 AdamW needs chunk_elems == 128");
  if (!is_fp8(a->state_dtype) || !is_fp8(v_dtype))
    return fail(MMUON_EINVAL, "FP8 AdamW needs F8E4M3 or F8E5M2 states (got %d, %d)", a->state_dtype, v_dtype);
  if (int rc = check_expand_min(expand_min)) return rc;
  if (a->nchunks > 0 && meta == nullptr) return fail(MMUON_EINVAL, "null FP8 metadata table");
  mmuon::AdamWArgs k = adamw_args(a);
  k.fp8 = meta;
  k.have_state = have_state ? 1 : 0;
  k.emin = expand_min;
  k.inv_sqrt_bc2 = 1.0f / a->sqrt_bc2;
  k.fast_quot = double(a->eps) * double(a->sqrt_bc2) >= 0x1p-37 && std::isfinite(k.inv_sqrt_bc2) ? 1 : 0;
  if (mmuon::launch_adamw_fp8(k, a->param_dtype, a->grad_dtype, a->state_dtype, v_dtype,
                              static_cast<hipStream_t>(stream)))
    return fail(MMUON_EINVAL, "unsupported FP8 AdamW dtypes param=%d grad=%d", a->param_dtype, a->grad_dtype);
  return check_launch("mmuon_adamw_fp8");
}

int mmuon_fp8_quantize(const float* value, uint8_t* codes, float* scale, float* expand, float* sqrt_minmax,
                       int64_t numel, int32_t signed_, int32_t fp8_dtype, float expand_min, void* stream) {
  if (numel < 0) return fail(MMUON_EINVAL, "negative numel");
  if (numel > 0 && (!value || !codes || !scale || !expand || !sqrt_minmax))
    return fail(MMUON_EINVAL, "null codec pointer");
  if (!is_fp8(fp8_dtype)) return fail(MMUON_EINVAL, "fp8_dtype must be MMUON_F8E4M3 or MMUON_F8E5M2");
  if (int rc = check_expand_min(expand_min)) return rc;
  if ((numel + 127) / 128 / 32 > 0x7fffffff) return fail(MMUON_ERANGE, "tensor too large");
  mmuon::launch_fp8_quantize(value, codes, scale, expand, sqrt_minmax, numel, signed_ != 0, fp8_dtype, expand_min,
                             static_cast<hipStream_t>(stream));
  return check_launch("mmuon_fp8_quantize");
}

int mmuon_fp8_dequantize(const uint8_t* codes, const float* scale, const float* expand,
                         const float* sqrt_minmax, float* out, int64_t numel, int32_t signed_,
                         int32_t fp8_dtype, void* stream) {
  if (numel < 0) return fail(MMUON_EINVAL, "negative numel");
  if (numel > 0 && (!out || !codes || !scale || !expand || !sqrt_minmax))
    return fail(MMUON_EINVAL, "null codec pointer");
  if (!is_fp8(fp8_dtype)) return fail(MMUON_EINVAL, "fp8_dtype must be MMUON_F8E4M3 or MMUON_F8E5M2");
  if ((numel + 127) / 128 / 32 > 0x7fffffff) return fail(MMUON_ERANGE, "tensor too large");
  mmuon::launch_fp8_dequantize(codes, scale, expand, sqrt_minmax, out, numel, signed_ != 0, fp8_dtype,
                               static_cast<hipStream_t>(stream));
  return check_launch("mmuon_fp8_dequantize");
}

int mmuon_grad_clip_coef(const mmuon_grad_norm_args* a, void* stream) {
  if (int rc = mmuon::check_grad_norm_args(a, true)) return rc;
  mmuon::launch_grad_clip_coef(*a, static_cast<hipStream_t>(stream));
  return check_launch("mmuon_grad_clip_coef");
}

}  // extern "C"

namespace {

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

int check_butterfly(const mmuon_butterfly_args* a, bool bwd) {
  if (a == nullptr) return fail(MMUON_EINVAL, "null butterfly arguments");
  if (a->dtype != MMUON_BF16) return fail(MMUON_EINVAL, "butterfly: dtype must be MMUON_BF16 (got %d)", a->dtype);
  const int nb = a->nblocks;
  if (nb != 1 && nb != 2 && nb != 4 && nb != 8 && nb != 16)
    return fail(MMUON_EINVAL, "butterfly: nblocks must be 1, 2, 4, 8 or 16 (got %d)", nb);
  if (a->q <= 0 || a->p <= 0 || a->s <= 0 || a->q % 8 || a->p % 8 || a->s % 8)
    return fail(MMUON_EINVAL, "butterfly: block sides must be positive multiples of 8 (q %d, p %d, s %d)", a->q, a->p,
                a->s);
  if ((a->q / nb) % 32 != 0 || a->q % nb != 0)
    return fail(MMUON_EINVAL, "butterfly: q / nblocks must be a multiple of 32 (q %d, nblocks %d)", a->q, nb);
  if (a->q >= (1 << 16) || a->p >= (1 << 16) || a->s >= (1 << 16))
    return fail(MMUON_ERANGE, "butterfly: block sides beyond 65535");
  if (a->tokens < 0 || a->tokens >= (int64_t(1) << 24))
    return fail(MMUON_ERANGE, "butterfly: tokens must be in [0, 2^24) (got %lld)", (long long)a->tokens);
  // per-lane offsets of a tile stay below 2^31: 256 rows of x, dout or out1
  // and 32 token rows x the planes of the intermediate
  const int64_t pitch = int64_t(std::max({nb * a->p, nb * a->s, a->q})) * 2;
  if (256 * pitch >= (int64_t(1) << 31) || int64_t(nb) * a->tokens * a->q * 2 >= (int64_t(1) << 31))
    return fail(MMUON_ERANGE, "butterfly: tensors beyond the kernels' 32-bit tile offsets");
  // token-sized tensors may be empty (null) when tokens == 0
  auto bad = [&](const void* p, bool per_token) {
    return (p == nullptr && !(per_token && a->tokens == 0)) || !aligned16(p);
  };
  if (bad(a->w1, false) || bad(a->w2, false) || bad(a->x, true) || bad(a->out1, true))
    return fail(MMUON_EINVAL, "butterfly: null or unaligned input pointer");
  if (!bwd) {
    if (bad(a->out, true)) return fail(MMUON_EINVAL, "butterfly: null or unaligned out");
    return MMUON_OK;
  }
  if (bad(a->dout, true) || bad(a->dx, true) || bad(a->dw1, false) || bad(a->dw2, false) || bad(a->workspace, false))
    return fail(MMUON_EINVAL, "butterfly: null or unaligned backward pointer");
  if ((reinterpret_cast<uintptr_t>(a->workspace) & 255) != 0)
    return fail(MMUON_EINVAL, "butterfly: workspace must be 256-B aligned");
  if (a->workspace_bytes < mmuon::butterfly_workspace(*a))
    return fail(MMUON_EINVAL, "butterfly: workspace of %zu bytes, %zu needed", a->workspace_bytes,
                mmuon::butterfly_workspace(*a));
  return MMUON_OK;
}

}  // namespace

extern "C" {

size_t mmuon_butterfly_workspace(const mmuon_butterfly_args* a) {
  if (a == nullptr || a->nblocks <= 0 || a->q <= 0 || a->p <= 0 || a->s <= 0 || a->tokens < 0) return 0;
  return mmuon::butterfly_workspace(*a);
}

int mmuon_butterfly_fwd(const mmuon_butterfly_args* a, void* stream) {
  if (int rc = check_butterfly(a, false)) return rc;
  mmuon::launch_butterfly_fwd(*a, static_cast<hipStream_t>(stream));
  return check_launch("butterfly forward");
}

int mmuon_butterfly_bwd(const mmuon_butterfly_args* a, void* stream) {
  if (int rc = check_butterfly(a, true)) return rc;
  mmuon::launch_butterfly_bwd(*a, static_cast<hipStream_t>(stream));
  return check_launch("butterfly backward");
}

}  // extern "C"
