/*
 * mmuon.h -- C ABI of libmmuon.so, the MI355X (gfx950) implementation of the
 * Monarch-Muon optimizer step (and of the Monarch butterfly multiply whose
 * backward produces the gradients the step consumes).
 *
 * The reference has no native boundary on this path: its step is a sequence
 * of torch ops (membench/src/models/monarch/monarch_muon.py:140-208,
 * pretrain/src/models/monarch/monarch_muon.py:139-201,
 * pretrain/src/models/monarch/coat_state_muon.py:22-139).  Each entry point
 * below names the reference lines whose work it replaces.
 *
 * Conventions
 *  - All pointers inside descriptors are DEVICE addresses owned by the caller
 *    (torch allocates every tensor, table and workspace); the library keeps
 *    no device allocations and no state between calls.
 *  - Every launch is enqueued on the caller's stream; no call synchronises.
 *  - Return value 0 = success; a negative MMUON_E* code otherwise, with a
 *    message retrievable through mmuon_last_error() (thread-local).
 *  - Descriptors are read on the host during the call only.
 */
#ifndef MMUON_H
#define MMUON_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* element types */
enum {
  MMUON_F32 = 0,
  MMUON_BF16 = 1,
  MMUON_F8E4M3 = 2, /* OCP float8_e4m3fn payload, with per-128 fp32 metadata */
  MMUON_F8E5M2 = 3  /* OCP float8_e5m2 payload, with per-128 fp32 metadata   */
};

/* error codes */
enum {
  MMUON_OK = 0,
  MMUON_EINVAL = -1,   /* bad argument (shape, dtype, null pointer, alignment) */
  MMUON_EHIP = -2,     /* a HIP runtime call failed */
  MMUON_ERANGE = -3    /* size beyond what a kernel's indexing supports */
};

/* One Monarch block (one r x c slice of a (nb, r, c) factor). */
typedef struct mmuon_block_ref {
  void* param;       /* r*c elements, row-major, param dtype      */
  const void* grad;  /* r*c elements, grad dtype                  */
  void* buf;         /* r*c elements, momentum dtype (F32/BF16), or the
                        FP8 payload (e4m3 / e5m2) of the FP8-state path */
} mmuon_block_ref;

/* FP8 metadata of one block: per 128-element group of the block's slice of the
   flattened parameter (the groups never straddle blocks; see
   mmuon_fp8_momentum_pack). */
typedef struct mmuon_block_fp8 {
  float* scale;
  float* expand;
  float* sqrt_minmax;
} mmuon_block_fp8;

/* Workspace geometry of one same-shape group, from mmuon_ns_layout().
   Matrix layout inside the stacks: fp32 row-major; bf16 in 32-column panels,
   element (i, j) of an R-row matrix at (j / 32) * R * 32 + i * 32 + j % 32. */
typedef struct mmuon_ns_layout_t {
  int32_t m, n;        /* Newton-Schulz orientation: m = min(r,c), n = max(r,c) */
  int32_t mp, np_;     /* padded m, n (multiples of the kernels' tiles)          */
  int32_t nparts;      /* partial sums of squares per block                      */
  int32_t ns_dtype;    /* MMUON_BF16 or MMUON_F32                                */
  int64_t x_bytes;     /* one X stack  [N] x (mp x np_)                           */
  int64_t a_bytes;     /* one Gram stack [N] x (mp x mp)                          */
  int64_t part_bytes;  /* partial sums   [N][nparts] fp32                         */
} mmuon_ns_layout_t;

/* A same-shape group of blocks, in the reference's grouping order. */
#define MMUON_GROUP_ALIGNED16 1  /* every block pointer is 16-byte aligned */
typedef struct mmuon_group {
  int32_t rows, cols;            /* block shape as stored (r, c)                 */
  int32_t nblocks;               /* N                                            */
  int32_t param_dtype;           /* F32 / BF16                                   */
  int32_t grad_dtype;            /* F32 / BF16                                   */
  int32_t buf_dtype;             /* F32 / BF16 / F8E4M3 / F8E5M2                 */
  int32_t ns_dtype;              /* BF16 (membench copy) or F32 (pretrain copy)  */
  int32_t flags;                 /* MMUON_GROUP_* bits                           */
  const mmuon_block_ref* blocks; /* device table, N entries                      */
  const mmuon_block_fp8* fp8;    /* device table, N entries (FP8 path), or NULL  */
  void* x0;                      /* workspace: X stack  (layout.x_bytes)         */
  void* x1;                      /* workspace: X stack  (layout.x_bytes)         */
  void* a;                       /* workspace: Gram     (layout.a_bytes)         */
  void* p;                       /* workspace: polynomial (layout.a_bytes)       */
  float* partial;                /* workspace: layout.part_bytes                 */
  float* scale;                  /* workspace: N floats                          */
  const float* grad_scale;       /* device: gradient-clipping coefficient from
                                    mmuon_grad_clip_coef, or NULL (no clipping)  */
} mmuon_group;

/* Geometry and workspace sizes for a group of (rows x cols) blocks.
   Replaces nothing in the reference (the reference allocates implicitly in
   torch.cat / bmm: membench monarch_muon.py:161-164). */
int mmuon_ns_layout(int32_t rows, int32_t cols, int32_t ns_dtype, int64_t nblocks,
                    mmuon_ns_layout_t* out);

/* Heavy-ball momentum + stack + cast, in one pass over the group:
     buf <- momentum*buf + grad          (rounded to the buffer dtype per op;
                                          grad = dtype(grad * *grad_scale) when
                                          g->grad_scale is set)
     X   <- cast(buf) to ns_dtype, transposed when rows > cols, into g->x0
     scale[b] <- 1 / (||X_b||_F + 1e-7), the Frobenius normalisation factor
   Replaces membench monarch_muon.py:146-151 (_foreach_mul_/_foreach_add_),
   :161-163 (torch.cat + .to(bf16)), :38 (the norm's reduction) and :40-41
   (the transpose); pretrain monarch_muon.py:143-148,158. */
int mmuon_momentum_pack(const mmuon_group* g, float momentum, void* stream);

/* FP8-state variant of mmuon_momentum_pack: buf holds FP8 codes (buf_dtype
   MMUON_F8E4M3 or MMUON_F8E5M2) with the per-128 metadata of g->fp8;
   dequantize -> momentum -> stack/cast -> requantize with the codec's
   expand_min (> 0; COAT's default 16).  `have_state` = 0 treats the momentum
   as zeros (first step, where the reference creates it with zeros_like).
   Requires rows*cols % 128 == 0 (every 128-group of the flattened parameter
   inside one block; other shapes go through mmuon_fp8_dequantize, the plain
   pack and mmuon_fp8_quantize over the whole parameter).
   Replaces coat_state_muon.py:126-139 (dequantize/quantize_ around the step,
   :94-114) fused with the work of mmuon_momentum_pack. */
int mmuon_fp8_momentum_pack(const mmuon_group* g, float momentum, int32_t have_state,
                            float expand_min, void* stream);

/* Newton-Schulz over the group's stack (already packed into g->x0) followed by
   the weight update:
     X <- X / (||X||_F + 1e-7)  (norm from the packed partial sums)
     repeat iters: A = X X^T ; P = b A + c A A ; X = a X + P X
     param <- param + alpha * cast(X) (un-transposed), alpha = -lr*sqrt(r/c)
   coeffs = {a, b, c}.  The launches are the ops of mmuon_ns_plan(g->rows,
   g->cols, g->ns_dtype, iters, flags): the three-product chain (X ping-pongs
   between x0 and x1), or for bf16 groups with np_ >= 2 mp and iters == 5 the
   Gram form (see mmuon_ns_plan).  flags: MMUON_NS_NO_APPLY leaves the final X
   in the workspace stack named by the plan's last op (standard chain: x0 when
   iters is even, x1 otherwise; Gram form: x0) and does not touch params;
   MMUON_NS_STANDARD selects the three-product chain for every group;
   MMUON_NS_HOLD_LAST launches every op of the plan but the last (for groups
   sharing their launches: the last op, the apply, then runs per group through
   mmuon_ns_run_op).
   Replaces membench monarch_muon.py:36-50 (_newton_schulz_batched, with the
   norm at :38-39), :164-170 (cast back, split, _foreach_add_ apply);
   pretrain monarch_muon.py:36-50,159-165. */
#define MMUON_NS_NO_APPLY 1
#define MMUON_NS_STANDARD 2
#define MMUON_NS_HOLD_LAST 4
int mmuon_newton_schulz_apply(const mmuon_group* g, int32_t iters, const float coeffs[3],
                              float alpha, int32_t flags, void* stream);

/* One launch of a Newton-Schulz plan.  Buffers: the group's workspace stacks
   x0, x1 (m x n), a, p (m x m), the two m x m sub-stacks of each X stack
   (X*_S0 at its start, X*_S1 after N mp^2 elements; only when np_ >= 2 mp),
   and the parameters.  Kinds (bf16 stacks keep symmetric m x m matrices as
   their 256 x 256 tiles on and above the diagonal):
     SYRK     out = s^2 in0 in0^T            (in0 an X stack)
     POLY     out = a I + b in0 + c in0 in0
     SYMM     out = in0 in1                  (two symmetric stacks that commute;
                                              bf16 only)
     PX       out = s in0 in1                (in1 an X stack, out an X stack)
     PX_APPLY param += alpha cast(s in0 in1)  (un-transposed)
   s = the block's 1/(||X_0||_F + 1e-7) when `scaled`, else 1. */
enum {
  MMUON_NSOP_SYRK = 0,
  MMUON_NSOP_POLY = 1,
  MMUON_NSOP_PX = 2,
  MMUON_NSOP_PX_APPLY = 3,
  MMUON_NSOP_SYMM = 4
};
enum {
  MMUON_NSB_X0 = 0,
  MMUON_NSB_X1 = 1,
  MMUON_NSB_A = 2,
  MMUON_NSB_P = 3,
  MMUON_NSB_X0_S0 = 4,
  MMUON_NSB_X0_S1 = 5,
  MMUON_NSB_X1_S0 = 6,
  MMUON_NSB_X1_S1 = 7,
  MMUON_NSB_PARAM = 8
};
typedef struct mmuon_ns_op {
  int32_t kind;       /* MMUON_NSOP_*                                   */
  int32_t in0, in1;   /* MMUON_NSB_* operands (in1 unused by SYRK, POLY) */
  int32_t out;        /* MMUON_NSB_* output                             */
  int32_t scaled;     /* 1: the op applies the block's normalisation    */
  int32_t iteration;  /* the quintic iteration the op belongs to        */
} mmuon_ns_op;

/* The launch plan of mmuon_newton_schulz_apply for a group of (rows x cols)
   blocks: writes up to max_ops ops (none when ops is NULL) and returns their
   number, or a negative error code.  Three-product chain: SYRK, POLY, PX per
   iteration.  Gram form (ns_dtype BF16, np_ >= 2 mp, iters == 5, no
   MMUON_NS_STANDARD): X_k = Q_k X_0 with Q_k a polynomial in A_0 = X_0 X_0^T, so
     P_k = a I + b A_k + c A_k^2, Q_{k+1} = P_k Q_k, A_{k+1} = P_k (P_k A_k)
   run on m x m matrices; X is rebuilt once (X_3 = Q_3 X_0) and the last two
   iterations restart from A_3 = X_3 X_3^T.  Equal to the chain in exact
   arithmetic; it replaces the m x m x n products of the other iterations by
   m x m x m ones.  Same reference lines as mmuon_newton_schulz_apply
   (the iteration of monarch_muon.py:43-48 re-associated). */
int mmuon_ns_plan(int32_t rows, int32_t cols, int32_t ns_dtype, int32_t iters, int32_t flags,
                  mmuon_ns_op* ops, int32_t max_ops);

/* Run one op of a plan on group g (validates the op against the group's
   geometry: buffer kinds, overlaps, sub-stack room).  A plan's ops run in order
   on one stream are exactly mmuon_newton_schulz_apply; this entry exists so a
   caller can time or inspect each launch.  Same reference lines. */
int mmuon_ns_run_op(const mmuon_group* g, const mmuon_ns_op* op, const float coeffs[3], float alpha,
                    void* stream);

/* One stage of one Newton-Schulz iteration (stage 0 = Gram X X^T, 1 = polynomial,
   2 = X update; on the last iteration stage 2 also applies the weight update
   unless MMUON_NS_NO_APPLY).  With a bf16 group the polynomial stage stores
   P = a I + b A + c A A (the a X term rides on P's diagonal, added in fp32
   before P's bf16 rounding) and stage 2 computes X = P X; with an fp32 group it
   stores P = b A + c A A and stage 2 computes X = a X + P X.
   These are the ops of the three-product chain (the plan with
   MMUON_NS_STANDARD), which mmuon_newton_schulz_apply runs for groups outside
   the Gram form; this entry exists so a caller can time each kernel with its
   own events.  Same reference lines as mmuon_newton_schulz_apply. */
int mmuon_ns_stage(const mmuon_group* g, int32_t iteration, int32_t iters, int32_t stage,
                   const float coeffs[3], float alpha, int32_t flags, void* stream);

/* Embedded AdamW over a list of tensors (one launch). */
typedef struct mmuon_adamw_tensor {
  void* param;        /* numel elements, param dtype */
  const void* grad;   /* grad dtype                  */
  void* exp_avg;      /* state dtype (or e4m3 codes) */
  void* exp_avg_sq;   /* state dtype (or e4m3 codes) */
  int64_t numel;
} mmuon_adamw_tensor;

typedef struct mmuon_adamw_args {
  const mmuon_adamw_tensor* tensors; /* device table                                  */
  const int64_t* chunks;             /* device: per chunk (tensor << 40 | first elem)  */
  int64_t nchunks;
  int32_t chunk_elems;               /* elements per chunk (128 on the FP8 path)       */
  int32_t param_dtype, grad_dtype, state_dtype;
  int32_t apply_weight_decay;        /* weight_decay > 0                               */
  /* scalars as the reference forms them in double and hands to torch ops */
  float wd_factor;                   /* 1 - lr * weight_decay                          */
  float beta1, beta2;
  float one_minus_beta1, one_minus_beta2;
  float sqrt_bc2;                    /* sqrt(1 - beta2 ** step)                        */
  float eps;
  float neg_step_size;               /* -lr / (1 - beta1 ** step)                      */
  const float* grad_scale;           /* device clipping coefficient, or NULL           */
} mmuon_adamw_args;

/* Replaces membench monarch_muon.py:176-208 (foreach AdamW: decoupled weight
   decay, bias corrections, eps after sqrt(v)/sqrt(bc2)) and pretrain
   :171-201.  state_dtype F32 or BF16. */
int mmuon_adamw(const mmuon_adamw_args* a, void* stream);

/* FP8-state AdamW: exp_avg (signed, format a->state_dtype) and exp_avg_sq
   (unsigned, format v_dtype), each MMUON_F8E4M3 or MMUON_F8E5M2 (the
   reference's first_order_bit / second_order_bit), held with per-128 metadata
   of the flattened tensor (a tensor's last group may be short); chunk_elems
   must be 128 (one metadata group per chunk); expand_min > 0.
   have_state = 1: the moments are dequantized to fp32 and updated in fp32.
   have_state = 0: the moments are created in this step: they start from zero
   in the PARAMETER dtype and every moment op rounds to it (the wrapped step
   creates them with zeros_like(param)); the codes are not read.
   Replaces coat_state_muon.py:126-139 around membench :176-208 /
   pretrain :171-201. */
typedef struct mmuon_adamw_fp8_tensor {
  float* scale_m; float* expand_m; float* sqrt_minmax_m;
  float* scale_v; float* expand_v; float* sqrt_minmax_v;
} mmuon_adamw_fp8_tensor;
int mmuon_adamw_fp8(const mmuon_adamw_args* a, const mmuon_adamw_fp8_tensor* meta,
                    int32_t have_state, int32_t v_dtype, float expand_min, void* stream);

/* Stand-alone codec over one flat tensor (numel elements; the last 128-group
   may be short):
   quantize: fp32 values -> FP8 codes (fp8_dtype MMUON_F8E4M3 or MMUON_F8E5M2)
             + scale/expand/sqrt_minmax per 128-group, with expand_min > 0
   dequantize: the inverse.  Replaces coat_state_muon.py:94-114 (_quantize_kernel
   :46-91, _dequantize_kernel :22-43; formats :17).  signed_ = 1 for
   first-order states. */
int mmuon_fp8_quantize(const float* value, uint8_t* codes, float* scale, float* expand,
                       float* sqrt_minmax, int64_t numel, int32_t signed_, int32_t fp8_dtype,
                       float expand_min, void* stream);
int mmuon_fp8_dequantize(const uint8_t* codes, const float* scale, const float* expand,
                         const float* sqrt_minmax, float* out, int64_t numel,
                         int32_t signed_, int32_t fp8_dtype, void* stream);

/* Gradient-norm clipping folded into the step.  Computes, over the listed
   gradients (one dtype, F32 or BF16), what torch.nn.utils.clip_grad_norm_
   (norm_type 2) computes before it rescales them:
     norm_t = dtype(sqrt(sum g^2))          per tensor, fp32 accumulation
     total  = dtype(sqrt(sum norm_t^2))
     coef   = min(dtype(dtype(1 / dtype(total + 1e-6)) * max_norm), 1)
   (dtype(.) rounds to the gradients' dtype; torch evaluates `max_norm / t` as
   t.reciprocal() * max_norm), writes total and coef, and leaves
   the gradients untouched.  A group or AdamW launch whose grad_scale points at
   coef then reads every gradient as dtype(g * coef), the value torch's in-place
   rescale leaves in p.grad.  Chunks: tensor << 40 | first element, chunk_elems
   elements each, every tensor's chunks contiguous and in tensor order;
   first_chunk[t] = index of tensor t's first chunk, first_chunk[ntensors] =
   nchunks.  partial: nchunks floats, norms: ntensors floats (workspace).
   Replaces pretrain/src/optim/base.py:121-122 (clip_grad_norm_ before
   opt.step(); its in-place rescale pass over the gradients is not needed). */
typedef struct mmuon_grad_tensor {
  const void* grad;
  int64_t numel;
} mmuon_grad_tensor;
typedef struct mmuon_grad_norm_args {
  const mmuon_grad_tensor* tensors;  /* device table, ntensors entries */
  const int64_t* chunks;             /* device, nchunks entries        */
  const int64_t* first_chunk;        /* device, ntensors + 1 entries   */
  int64_t nchunks;
  int32_t ntensors;
  int32_t chunk_elems;
  int32_t grad_dtype;
  float max_norm;
  float* partial;
  float* norms;
  float* total;                      /* device, 1 float (out) */
  float* coef;                       /* device, 1 float (out) */
} mmuon_grad_norm_args;
int mmuon_grad_clip_coef(const mmuon_grad_norm_args* a, void* stream);

/* The same coefficient with no caller workspace: exactly mmuon_grad_clip_coef's
   kernels and results, with a->partial and a->norms ignored (pass NULL); the
   caller still passes the tables and the total / coef outputs.
   No counterpart in the reference.  It is for callers that cannot allocate
   device memory (code under HIP graph capture, tight training or serving
   loops, harnesses that forbid hipMalloc); this call allocates nothing.  The
   partial sums and norms live in a static array the library holds on each GPU
   until the process ends: MMUON_NOALLOC_SCRATCH_FLOATS floats (4 MiB), enough
   for (nchunks rounded up to 64) + ntensors; larger inputs return
   MMUON_ERANGE.  The stream must belong to the current device.  Calls on one
   stream are ordered; calls that overlap on one GPU (several streams or
   threads) share the array and race.  The first call on each device looks up
   the array's device address (hipGetSymbolAddress): make that call outside
   graph capture; later calls can be captured and replayed (the captured
   launches hold the table, output and gradient addresses of that call). */
#define MMUON_NOALLOC_SCRATCH_FLOATS (1 << 20)
int mmuon_grad_clip_coef_noalloc(const mmuon_grad_norm_args* a, void* stream);

/* Monarch butterfly multiply, the layer step that produces the (nb, r, c)
   gradients the optimizer consumes.  w1 (nblocks, q, p) and w2 (nblocks, s, q)
   are a MonarchLinear's blkdiag1 / blkdiag2 (k = l = nblocks, r = q);
   x (tokens, nblocks * p) its padded input.  bf16 throughout, fp32
   accumulation, every product rounded to bf16 as the reference's bmms round.
     out1[ll][b][i]  = riffle of x[b][kk] . w1[kk]^T  (nblocks, tokens, q),
                       the intermediate saved for the backward;
     out[b][ll][j]   = out1[ll][b] . w2[ll][j]       (tokens, nblocks, s),
                       the blocked output (the caller's view
                       out.transpose(1, 2).reshape(tokens, s * nblocks) is the
                       layer's feature order).
   Requirements: p, q, s multiples of 8; q / nblocks a multiple of 32;
   nblocks in {1, 2, 4, 8, 16}; 1 <= tokens < 2^24 (0 allowed); every pointer
   16-B aligned, tensors contiguous.  The tensors must not overlap. */
typedef struct mmuon_butterfly_args {
  int64_t tokens;
  int32_t nblocks;
  int32_t q, p, s;
  int32_t dtype;          /* MMUON_BF16 */
  const void* x;          /* (tokens, nblocks * p)   */
  const void* w1;         /* (nblocks, q, p)         */
  const void* w2;         /* (nblocks, s, q)         */
  void* out;              /* forward out: (tokens, nblocks, s)  */
  void* out1;             /* forward out / backward in: (nblocks, tokens, q) */
  const void* dout;       /* backward in: (tokens, nblocks, s)  */
  void* dx;               /* backward out: (tokens, nblocks * p) */
  void* dw1;              /* backward out: (nblocks, q, p) */
  void* dw2;              /* backward out: (nblocks, s, q) */
  void* workspace;        /* backward: mmuon_butterfly_workspace() bytes, 256-B aligned */
  size_t workspace_bytes;
} mmuon_butterfly_args;
/* Forward.  Replaces pretrain/src/models/monarch/monarch_ops.py:23-46
   (_butterfly_fwd_blocked / monarch::butterfly_blk: two bmms with the riffle of
   monarch_riffle.py:13-57 between them); out1 is written in riffled order by
   the first product, so no separate riffle pass runs. */
int mmuon_butterfly_fwd(const mmuon_butterfly_args* a, void* stream);
/* Backward: dx, dw1, dw2 from x, w1, w2, out1 and dout.  Replaces
   pretrain/src/models/monarch/monarch_ops.py:57-82 (monarch::butterfly_blk_bwd:
   four bmms and the unriffle of monarch_riffle.py:60-107); the unriffle is
   folded into the addressing of the products that read it. */
int mmuon_butterfly_bwd(const mmuon_butterfly_args* a, void* stream);
/* Workspace bytes the backward needs for these shapes (x, pointers unused). */
size_t mmuon_butterfly_workspace(const mmuon_butterfly_args* a);

/* Thread-local message of the last failing call ("" if none). */
const char* mmuon_last_error(void);

/* ABI version: bumped on any change to this header. */
int mmuon_abi_version(void);

#ifdef __cplusplus
}
#endif
#endif /* MMUON_H */
