// extern "C" entry points of libmmuon.so (declared in include/mmuon.h).
// Argument validation, workspace geometry, stage sequencing; every launch on
// the caller's stream, no synchronisation, no device allocation.
#include <stdarg.h>
#include <stdio.h>

#include <algorithm>
#include <string>

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
  }
  return 0;
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

int mmuon_abi_version(void) { return 5; }

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

int mmuon_fp8_momentum_pack(const mmuon_group* g, float momentum, int32_t have_state, void* stream) {
  Geometry geo;
  if (int rc = check_group(g, geo)) return rc;
  if (g->buf_dtype != MMUON_F8E4M3) return fail(MMUON_EINVAL, "buf dtype must be MMUON_F8E4M3");
  if (g->fp8 == nullptr) return fail(MMUON_EINVAL, "null FP8 metadata table");
  if ((int64_t(g->rows) * g->cols) % 128 != 0)
    return fail(MMUON_EINVAL, "FP8 momentum needs rows*cols %% 128 == 0 (got %d x %d)", g->rows, g->cols);
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const int nparts = mmuon::fp8_pack_nparts(g->rows, g->cols, geo.transposed);
  mmuon::PackArgs a = pack_args(g, geo, momentum, nparts);
  if (mmuon::launch_fp8_pack(a, g->fp8, g->rows, g->cols, g->grad_dtype, g->ns_dtype, geo.transposed,
                             have_state ? 1 : 0, s))
    return fail(MMUON_EINVAL, "unsupported dtype combination grad=%d ns=%d", g->grad_dtype, g->ns_dtype);
  mmuon::launch_block_scale(g->partial, nparts, g->scale, g->nblocks, g->ns_dtype == MMUON_BF16, s);
  return check_launch("mmuon_fp8_momentum_pack");
}

}  // extern "C"

namespace {

// Launch one stage of one iteration; X ping-pongs between x0 (even iterations'
// input) and x1.
int ns_stage(const mmuon_group* g, const Geometry& geo, int it, int iters, int stage,
             const float coeffs[3], float alpha, int flags, hipStream_t s) {
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
  void* cur = (it & 1) ? g->x1 : g->x0;
  void* nxt = (it & 1) ? g->x0 : g->x1;
  const float* sc = it == 0 ? g->scale : nullptr;
  int kstage = stage;
  switch (stage) {
    case 0:
      a.scale = sc;
      a.x_in = cur;
      a.out = g->a;
      kstage = mmuon::NS_SYRK;
      break;
    case 1:
      a.a_in = g->a;
      a.out = g->p;
      kstage = mmuon::NS_POLY;
      break;
    case 2: {
      a.scale = sc;
      a.a_in = g->p;
      a.x_in = cur;
      a.out = nxt;
      const bool apply = !(flags & MMUON_NS_NO_APPLY) && it + 1 == iters;
      kstage = apply ? mmuon::NS_PX_APPLY : mmuon::NS_PX;
      break;
    }
    default:
      return fail(MMUON_EINVAL, "stage must be 0, 1 or 2 (got %d)", stage);
  }
  if (mmuon::launch_ns_stage(a, kstage, g->ns_dtype, g->param_dtype, s))
    return fail(MMUON_EINVAL, "no Newton-Schulz kernel for ns dtype %d / param dtype %d", g->ns_dtype,
                g->param_dtype);
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

int mmuon_newton_schulz_apply(const mmuon_group* g, int32_t iters, const float coeffs[3], float alpha,
                              int32_t flags, void* stream) {
  Geometry geo;
  if (int rc = check_ns(g, geo, iters, coeffs)) return rc;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  for (int it = 0; it < iters; ++it)
    for (int st = 0; st < 3; ++st)
      if (int rc = ns_stage(g, geo, it, iters, st, coeffs, alpha, flags, s)) return rc;
  return check_launch("mmuon_newton_schulz_apply");
}

int mmuon_ns_stage(const mmuon_group* g, int32_t iteration, int32_t iters, int32_t stage,
                   const float coeffs[3], float alpha, int32_t flags, void* stream) {
  Geometry geo;
  if (int rc = check_ns(g, geo, iters, coeffs)) return rc;
  if (iteration < 0 || iteration >= iters)
    return fail(MMUON_EINVAL, "iteration %d outside [0, %d)", iteration, iters);
  if (int rc = ns_stage(g, geo, iteration, iters, stage, coeffs, alpha, flags, static_cast<hipStream_t>(stream)))
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
                    void* stream) {
  if (int rc = check_adamw(a)) return rc;
  if (a->chunk_elems != 128) return fail(MMUON_EINVAL, "FP8 AdamW needs chunk_elems == 128");
  if (a->state_dtype != MMUON_F8E4M3) return fail(MMUON_EINVAL, "FP8 AdamW needs state dtype F8E4M3");
  if (a->nchunks > 0 && meta == nullptr) return fail(MMUON_EINVAL, "null FP8 metadata table");
  mmuon::AdamWArgs k = adamw_args(a);
  k.fp8 = meta;
  k.have_state = have_state ? 1 : 0;
  if (mmuon::launch_adamw_fp8(k, a->param_dtype, a->grad_dtype, static_cast<hipStream_t>(stream)))
    return fail(MMUON_EINVAL, "unsupported FP8 AdamW dtypes param=%d grad=%d", a->param_dtype, a->grad_dtype);
  return check_launch("mmuon_adamw_fp8");
}

int mmuon_fp8_quantize(const float* value, uint8_t* codes, float* scale, float* expand, float* sqrt_minmax,
                       int64_t numel, int32_t signed_, void* stream) {
  if (numel < 0) return fail(MMUON_EINVAL, "negative numel");
  if (numel > 0 && (!value || !codes || !scale || !expand || !sqrt_minmax))
    return fail(MMUON_EINVAL, "null codec pointer");
  if ((numel + 127) / 128 / 4 > 0x7fffffff) return fail(MMUON_ERANGE, "tensor too large");
  mmuon::launch_fp8_quantize(value, codes, scale, expand, sqrt_minmax, numel, signed_ != 0,
                             static_cast<hipStream_t>(stream));
  return check_launch("mmuon_fp8_quantize");
}

int mmuon_fp8_dequantize(const uint8_t* codes, const float* scale, const float* expand,
                         const float* sqrt_minmax, float* out, int64_t numel, int32_t signed_,
                         void* stream) {
  if (numel < 0) return fail(MMUON_EINVAL, "negative numel");
  if (numel > 0 && (!out || !codes || !scale || !expand || !sqrt_minmax))
    return fail(MMUON_EINVAL, "null codec pointer");
  if (numel / 256 > 0x7fffffff) return fail(MMUON_ERANGE, "tensor too large");
  mmuon::launch_fp8_dequantize(codes, scale, expand, sqrt_minmax, out, numel, signed_ != 0,
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
