// Host-side launch interfaces shared between the kernel files and the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/mmuon.h"

namespace mmuon {

struct PackArgs {
  const mmuon_block_ref* blocks;
  void* x;          // X stack [N][mp][np] in the NS dtype
  float* partial;   // [N][nparts]
  int N;
  int m, n;         // NS orientation (m = min(rows, cols))
  int mp, np;       // padded extents of the X stack
  int nparts;
  float mu;
  int vec;          // 8-wide vector access is valid for every block
  const float* gscale;  // gradient-clipping coefficient (device), or null
};

int pack_nparts(int mp, int np_, bool transposed);
int launch_pack(const PackArgs& a, int grad_dtype, int buf_dtype, int x_dtype, bool transposed,
                hipStream_t s);
void launch_block_scale(const float* partial, int nparts, float* scale, int N, bool bf16_norm,
                        hipStream_t s);

// Newton-Schulz stage kernels -------------------------------------------------
enum NsStage { NS_SYRK = 0, NS_POLY = 1, NS_PX = 2, NS_PX_APPLY = 3, NS_SYMM = 4 };

struct NsArgs {
  const void* x_in;   // X stack, N x (mp x np)
  const void* a_in;   // Gram / polynomial stack, N x (mp x mp)
  const void* b_in;   // SYMM: the column operand, a second symmetric N x (mp x mp) stack
  void* out;          // stage output
  const float* scale; // per-block 1/(||X||+eps) for the first iteration, else null
  const mmuon_block_ref* blocks;  // apply stage: parameter pointers
  int N, m, n, mp, np;
  int kx;             // contraction extent of the Gram product (n rounded to the K tile)
  float ca, cb, cc;   // quintic coefficients
  float alpha;        // apply: -lr * sqrt(rows / cols)
  int transposed;     // rows > cols
  int vec;            // apply: every parameter block is 16-B aligned
};

// geometry helpers (tile sizes of the kernels)
int ns_tile_m(int ns_dtype);
int ns_tile_n(int ns_dtype);
int ns_tile_k(int ns_dtype);
int launch_ns_stage(const NsArgs& a, int stage, int ns_dtype, int param_dtype, hipStream_t s);

// AdamW ---------------------------------------------------------------------
struct AdamWArgs {
  const mmuon_adamw_tensor* tensors;
  const int64_t* chunks;
  int64_t nchunks;
  int chunk_elems;
  float wd_factor;      // 1 - lr * weight_decay
  int apply_wd;         // weight_decay > 0
  float beta1, one_minus_beta1, beta2, one_minus_beta2;
  float sqrt_bc2;       // sqrt(1 - beta2^t)
  float eps;
  float neg_step_size;  // -lr / (1 - beta1^t)
  const mmuon_adamw_fp8_tensor* fp8;
  int have_state;
  float emin;           // FP8 states: expand_min of the codec
  const float* gscale;  // gradient-clipping coefficient (device), or null
  float inv_sqrt_bc2;   // FP8 states: fp32 1 / sqrt_bc2
  int fast_quot;        // FP8 states: hardware root and reciprocal (eps sqrt_bc2 >= 2^-37)
};
int launch_adamw(const AdamWArgs& a, int param_dtype, int grad_dtype, int state_dtype,
                 hipStream_t s);
int launch_adamw_fp8(const AdamWArgs& a, int param_dtype, int grad_dtype, int m_dtype, int v_dtype, hipStream_t s);

// Gradient-norm clipping coefficient --------------------------------------------
int launch_grad_clip_coef(const mmuon_grad_norm_args& a, hipStream_t s);
// argument checks shared by the two entry points (workspace: partial and norms
// must be given)
int check_grad_norm_args(const mmuon_grad_norm_args* a, bool workspace);

// Error reporting shared by the translation units: set the thread-local
// message of mmuon_last_error and return code; the status of the last launch.
int set_error(int code, const char* msg);
int launch_status(const char* what);

// Monarch butterfly multiply -------------------------------------------------------
size_t butterfly_workspace(const mmuon_butterfly_args& a);
int launch_butterfly_fwd(const mmuon_butterfly_args& a, hipStream_t s);
int launch_butterfly_bwd(const mmuon_butterfly_args& a, hipStream_t s);

// Gradient-clipping coefficient of a launch (gscale: device pointer, or null
// when not clipping), read once per thread: the per-element form would test
// the pointer in every element (a branch each) and, after the thread's first
// store, reload the coefficient with a wait on every memory access in flight.
struct GradClip {
  bool on;
  float c;
};
__device__ __forceinline__ GradClip grad_clip(const float* gscale) {
  return gscale != nullptr ? GradClip{true, *gscale} : GradClip{false, 1.f};
}
// Gradient as the step reads it: dtype(g * c) when clipping, else g.
template <class TG>
__device__ __forceinline__ float clipped(float g, GradClip k) {
  return k.on ? TG::round(g * k.c) : g;
}
template <class TG, int N>
__device__ __forceinline__ void clip_grads(float (&g)[N], GradClip k) {
  if (k.on) {
#pragma unroll
    for (int i = 0; i < N; ++i) g[i] = TG::round(g[i] * k.c);
  }
}

// FP8 codec (fp8_dtype: MMUON_F8E4M3 or MMUON_F8E5M2; emin: expand_min) -------
int launch_fp8_quantize(const float* v, uint8_t* q, float* sc, float* ex, float* smm, int64_t numel, bool sgn,
                        int fp8_dtype, float emin, hipStream_t s);
int launch_fp8_dequantize(const uint8_t* q, const float* sc, const float* ex, const float* smm, float* out,
                          int64_t numel, bool sgn, int fp8_dtype, hipStream_t s);
int fp8_pack_nparts(int rows, int cols, bool transposed);
int launch_fp8_pack(const PackArgs& a, const mmuon_block_fp8* meta, int rows, int cols, int grad_dtype, int x_dtype,
                    int fp8_dtype, bool transposed, int have_state, float emin, hipStream_t s);

}  // namespace mmuon
