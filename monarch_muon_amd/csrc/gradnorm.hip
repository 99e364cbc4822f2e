// Gradient-norm clipping coefficient, folded into the step.
//
// pretrain/src/optim/base.py:121-122 calls torch.nn.utils.clip_grad_norm_
// (norm_type 2) right before opt.step(): per-tensor norms, the norm of those
// norms, coef = min(max_norm / (total + 1e-6), 1) in the gradients' dtype, and
// an in-place rescale of every gradient.  Here three small launches produce
// total and coef on the device (no host round trip); the step's kernels then
// read each gradient as dtype(g * coef), so the rescale pass is not needed.
// Reductions run in a fixed order, so the result does not vary between runs.
// Algorithmic HBM traffic: one read of every gradient.
#include <stdio.h>

#include <mutex>

#include "common.hpp"
#include "kernels.hpp"

namespace mmuon {

constexpr int GN_NT = 256;

// One workgroup per chunk: fp32 sum of squares of its elements.
template <class TG>
__global__ __launch_bounds__(GN_NT) void grad_sumsq_kernel(const mmuon_grad_tensor* tensors, const int64_t* chunks,
                                                           int chunk_elems, float* partial) {
  __shared__ float red[GN_NT / 64];
  const int64_t code = chunks[blockIdx.x];
  const mmuon_grad_tensor T = tensors[int(code >> 40)];
  const int64_t start = code & ((int64_t(1) << 40) - 1);
  const int64_t end = min(T.numel, start + int64_t(chunk_elems));
  const auto* g = reinterpret_cast<const typename TG::storage*>(T.grad);
  float ss = 0.f;
  int64_t tail = start;
  if ((reinterpret_cast<uintptr_t>(g + start) & 15) == 0) {
    const int64_t stop = start + ((end - start) & ~int64_t(7));
    for (int64_t i = start + int64_t(threadIdx.x) * 8; i < stop; i += GN_NT * 8) {
      float v[8];
      Vec8<TG>::load(g + i, v);
#pragma unroll
      for (int k = 0; k < 8; ++k) ss = fmaf(v[k], v[k], ss);
    }
    tail = stop;
  }
  for (int64_t i = tail + threadIdx.x; i < end; i += GN_NT) {
    const float v = TG::load(g, i);
    ss = fmaf(v, v, ss);
  }
  const float tot = block_sum<GN_NT>(ss, red);
  if (threadIdx.x == 0) partial[blockIdx.x] = tot;
}

// One workgroup per tensor: norm_t = dtype(sqrt(sum of its chunks' partials)).
template <class TG>
__global__ __launch_bounds__(GN_NT) void grad_tensor_norm_kernel(const int64_t* first_chunk, const float* partial,
                                                                 float* norms) {
  __shared__ float red[GN_NT / 64];
  const int t = blockIdx.x;
  const int64_t c0 = first_chunk[t], c1 = first_chunk[t + 1];
  float s = 0.f;
  for (int64_t c = c0 + threadIdx.x; c < c1; c += GN_NT) s += partial[c];
  const float tot = block_sum<GN_NT>(s, red);
  if (threadIdx.x == 0) norms[t] = TG::round(sqrtf(tot));
}

// total = dtype(sqrt(sum norm_t^2)); coef = min(max_norm / dtype(total + 1e-6), 1), the
// division evaluated as torch evaluates `float / tensor`: dtype(dtype(1 / x) * max_norm).
template <class TG>
__global__ __launch_bounds__(GN_NT) void clip_coef_kernel(const float* norms, int ntensors, float max_norm,
                                                          float* total, float* coef) {
  __shared__ float red[GN_NT / 64];
  float s = 0.f;
  for (int t = threadIdx.x; t < ntensors; t += GN_NT) s = fmaf(norms[t], norms[t], s);
  const float tot = block_sum<GN_NT>(s, red);
  if (threadIdx.x == 0) {
    const float n = TG::round(sqrtf(tot));
    const float r = TG::round(1.0f / TG::round(n + 1e-6f));
    const float c = TG::round(r * max_norm);
    total[0] = n;
    coef[0] = fminf(c, 1.0f);
  }
}

int launch_grad_clip_coef(const mmuon_grad_norm_args& a, hipStream_t s) {
  if (a.nchunks > 0) {
    if (a.grad_dtype == MMUON_BF16)
      hipLaunchKernelGGL(grad_sumsq_kernel<BF16T>, dim3(unsigned(a.nchunks)), dim3(GN_NT), 0, s, a.tensors, a.chunks,
                         a.chunk_elems, a.partial);
    else
      hipLaunchKernelGGL(grad_sumsq_kernel<F32T>, dim3(unsigned(a.nchunks)), dim3(GN_NT), 0, s, a.tensors, a.chunks,
                         a.chunk_elems, a.partial);
  }
  if (a.ntensors > 0) {
    if (a.grad_dtype == MMUON_BF16)
      hipLaunchKernelGGL(grad_tensor_norm_kernel<BF16T>, dim3(unsigned(a.ntensors)), dim3(GN_NT), 0, s,
                         a.first_chunk, a.partial, a.norms);
    else
      hipLaunchKernelGGL(grad_tensor_norm_kernel<F32T>, dim3(unsigned(a.ntensors)), dim3(GN_NT), 0, s,
                         a.first_chunk, a.partial, a.norms);
  }
  if (a.grad_dtype == MMUON_BF16)
    hipLaunchKernelGGL(clip_coef_kernel<BF16T>, dim3(1), dim3(GN_NT), 0, s, a.norms, a.ntensors, a.max_norm,
                       a.total, a.coef);
  else
    hipLaunchKernelGGL(clip_coef_kernel<F32T>, dim3(1), dim3(GN_NT), 0, s, a.norms, a.ntensors, a.max_norm,
                       a.total, a.coef);
  return 0;
}

// ---------------------------------------------------------------------------
// mmuon_grad_clip_coef_noalloc: the same three launches with the per-chunk
// partial sums and the per-tensor norms in `scratch`, a file-scope device
// array, instead of caller workspace.  Each GPU the library runs on holds its
// own copy (MMUON_NOALLOC_SCRATCH_FLOATS floats) until the process ends; in
// host code `scratch` names a host-side stand-in, so its device address is
// looked up once per device (hipGetSymbolAddress, with that device current)
// and only that address is handed to kernels.  Every partial and norm is
// written before it is read within one call, so nothing needs clearing; calls
// that overlap on one GPU (other streams, other threads) share the array and
// race.
// ---------------------------------------------------------------------------
static __device__ __align__(256) float scratch[MMUON_NOALLOC_SCRATCH_FLOATS];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch_ptr[kMaxDevices];  // device address of `scratch` per device, once looked up

int scratch_address(int dev, float** out) {
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      char msg[256];
      snprintf(msg, sizeof msg, "hipGetSymbolAddress(scratch) on device %d: %s", dev, hipGetErrorString(e));
      return set_error(MMUON_EHIP, msg);
    }
    g_scratch_ptr[dev] = static_cast<float*>(p);
  }
  *out = g_scratch_ptr[dev];
  return MMUON_OK;
}

}  // namespace
}  // namespace mmuon

extern "C" int mmuon_grad_clip_coef_noalloc(const mmuon_grad_norm_args* a, void* stream) {
  using namespace mmuon;
  if (int rc = check_grad_norm_args(a, false)) return rc;
  // partials [0, nchunks), norms from the next 256-B boundary
  const int64_t norms_at = (a->nchunks + 63) / 64 * 64;
  const int64_t need = norms_at + a->ntensors;
  char msg[256];
  if (need > MMUON_NOALLOC_SCRATCH_FLOATS) {
    snprintf(msg, sizeof msg,
             "needs %lld floats of scratch (%lld chunks, %d tensors); the no-allocation entry point holds %d",
             (long long)need, (long long)a->nchunks, a->ntensors, MMUON_NOALLOC_SCRATCH_FLOATS);
    return set_error(MMUON_ERANGE, msg);
  }
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    snprintf(msg, sizeof msg, "hipGetDevice: %s", hipGetErrorString(e));
    return set_error(MMUON_EHIP, msg);
  }
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (s != nullptr) {
    hipDevice_t sd = 0;
    e = hipStreamGetDevice(s, &sd);
    if (e != hipSuccess) {
      snprintf(msg, sizeof msg, "hipStreamGetDevice: %s", hipGetErrorString(e));
      return set_error(MMUON_EHIP, msg);
    }
    if (int(sd) != dev) {
      snprintf(msg, sizeof msg, "the stream belongs to device %d but device %d is current", int(sd), dev);
      return set_error(MMUON_EINVAL, msg);
    }
  }
  if (dev < 0 || dev >= kMaxDevices) return set_error(MMUON_ERANGE, "device index beyond 63");
  float* base = nullptr;
  if (int rc = scratch_address(dev, &base)) return rc;
  mmuon_grad_norm_args k = *a;
  k.partial = base;
  k.norms = base + norms_at;
  launch_grad_clip_coef(k, s);
  return launch_status("mmuon_grad_clip_coef_noalloc");
}
