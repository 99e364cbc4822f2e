// HBM streaming probes: the read, write and copy bandwidth this GPU sustains
// for 16-B vector accesses, the ceiling the momentum pack and AdamW (both
// HBM-bound streaming kernels) are measured against.  Not part of the
// optimizer step.
#include <stdio.h>

#include "common.hpp"
#include "kernels.hpp"

namespace mmuon {
namespace {

constexpr int SP_NT = 256;
constexpr int SP_UNROLL = 4;

__device__ __forceinline__ uint4 ld16(const uint4* p, bool nt) {
  return nt ? load16_nt(p) : *p;
}
__device__ __forceinline__ void st16(uint4* p, const uint4& v, bool nt) {
  if (nt) store16_nt(p, v);
  else *p = v;
}

// Data written by the write probe: a 64-bit multiplicative hash of the chunk
// index, so that the stored bits look random (HBM power depends on the data).
__device__ __forceinline__ uint4 pattern(int64_t i) {
  const uint64_t h = uint64_t(i + 1) * 0x9E3779B97F4A7C15ull;
  const uint64_t g = (h ^ (h >> 29)) * 0xBF58476D1CE4E5B9ull;
  return make_uint4(uint32_t(h >> 32), uint32_t(g), uint32_t(g >> 32), uint32_t(h) ^ uint32_t(g >> 17));
}

// KIND 0: read n16 chunks of src; 1: write n16 chunks of dst; 2: copy.
// Grid-stride, SP_UNROLL independent accesses in flight per thread.  The read
// probe folds what it reads into one value per thread and stores it only if it
// equals an improbable pattern, so the loads cannot be dropped.
template <int KIND, bool NTA>
__global__ __launch_bounds__(SP_NT) void stream_probe_kernel(uint4* __restrict__ dst, const uint4* __restrict__ src,
                                                             int64_t n16) {
  const int64_t stride = int64_t(gridDim.x) * SP_NT;
  int64_t i = int64_t(blockIdx.x) * SP_NT + threadIdx.x;
  uint4 acc = make_uint4(0, 0, 0, 0);
  for (; i + (SP_UNROLL - 1) * stride < n16; i += SP_UNROLL * stride) {
    uint4 v[SP_UNROLL];
    if constexpr (KIND != 1) {
#pragma unroll
      for (int u = 0; u < SP_UNROLL; ++u) v[u] = ld16(src + i + u * stride, NTA);
    } else {
#pragma unroll
      for (int u = 0; u < SP_UNROLL; ++u) v[u] = pattern(i + u * stride);
    }
    if constexpr (KIND == 0) {
#pragma unroll
      for (int u = 0; u < SP_UNROLL; ++u) {
        acc.x ^= v[u].x; acc.y += v[u].y; acc.z ^= v[u].z; acc.w += v[u].w;
      }
    } else {
#pragma unroll
      for (int u = 0; u < SP_UNROLL; ++u) st16(dst + i + u * stride, v[u], NTA);
    }
  }
  for (; i < n16; i += stride) {
    if constexpr (KIND == 0) {
      const uint4 v = ld16(src + i, NTA);
      acc.x ^= v.x; acc.y += v.y; acc.z ^= v.z; acc.w += v.w;
    } else if constexpr (KIND == 1) {
      st16(dst + i, pattern(i), NTA);
    } else {
      st16(dst + i, ld16(src + i, NTA), NTA);
    }
  }
  if constexpr (KIND == 0) {
    if (acc.x == 0x9E3779B9u && acc.y == 0x7F4A7C15u && acc.z == 0xBF58476Du && acc.w == 0x1CE4E5B9u && dst)
      dst[int64_t(blockIdx.x) * SP_NT + threadIdx.x] = acc;
  }
}

template <int KIND>
void launch_probe(uint4* dst, const uint4* src, int64_t n16, bool nt, int grid, hipStream_t s) {
  if (nt) hipLaunchKernelGGL((stream_probe_kernel<KIND, true>), dim3(grid), dim3(SP_NT), 0, s, dst, src, n16);
  else hipLaunchKernelGGL((stream_probe_kernel<KIND, false>), dim3(grid), dim3(SP_NT), 0, s, dst, src, n16);
}

}  // namespace
}  // namespace mmuon

extern "C" int mmuon_hbm_stream(int32_t kind, void* dst, const void* src, int64_t bytes, int32_t nontemporal,
                                int32_t grid, void* stream) {
  using namespace mmuon;
  char msg[160];
  if (kind < 0 || kind > 2) return set_error(MMUON_EINVAL, "kind must be 0 (read), 1 (write) or 2 (copy)");
  if (bytes <= 0 || bytes % 16) return set_error(MMUON_EINVAL, "bytes must be a positive multiple of 16");
  if (grid < 1 || grid > (1 << 20)) return set_error(MMUON_EINVAL, "grid must be in [1, 2^20]");
  if ((kind != 1 && src == nullptr) || (kind != 0 && dst == nullptr)) return set_error(MMUON_EINVAL, "null buffer");
  if ((reinterpret_cast<uintptr_t>(dst) | reinterpret_cast<uintptr_t>(src)) % 16)
    return set_error(MMUON_EINVAL, "buffers must be 16-B aligned");
  // the read probe's improbable store lands in dst[0 .. grid * 256) when dst is given
  if (kind == 0 && dst != nullptr && int64_t(grid) * SP_NT * 16 > bytes) {
    snprintf(msg, sizeof msg, "read probe: dst must hold grid * 4096 bytes (%lld)", (long long)grid * SP_NT * 16);
    return set_error(MMUON_EINVAL, msg);
  }
  const int64_t n16 = bytes / 16;
  auto* d = static_cast<uint4*>(dst);
  const auto* sr = static_cast<const uint4*>(src);
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const bool nt = nontemporal != 0;
  if (kind == 0) launch_probe<0>(d, sr, n16, nt, grid, s);
  else if (kind == 1) launch_probe<1>(d, sr, n16, nt, grid, s);
  else launch_probe<2>(d, sr, n16, nt, grid, s);
  return launch_status("mmuon_hbm_stream");
}
