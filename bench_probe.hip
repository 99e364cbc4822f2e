// HBM streaming probes for bench.py (--hbm-ceiling, --data-energy): the read,
// write, copy, in-place update and momentum-pack-pattern bandwidth this GPU
// sustains for 16-B vector accesses, the ceilings the momentum pack and AdamW
// (both HBM-bound streaming kernels) are measured against.  Built as its own
// library (bench_probe.so), apart from libmmuon.so: it is not part of the
// optimizer step or of its C ABI.
#include <stdio.h>

#include <string>

#include "monarch_muon_amd/csrc/common.hpp"

namespace mmuon {
namespace {

thread_local std::string g_probe_err;

int set_error(int code, const char* msg) {
  g_probe_err = msg;
  return code;
}

int launch_status(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e == hipSuccess) return MMUON_OK;
  char msg[256];
  snprintf(msg, sizeof msg, "%s: %s", what, hipGetErrorString(e));
  return set_error(MMUON_EHIP, msg);
}

constexpr int SP_NT = 256;
constexpr int SP_UNROLL = 4;

__device__ __forceinline__ uint4 ld16(const uint4* p, bool nt) {
  return nt ? load16_nt(p) : *p;
}
__device__ __forceinline__ void st16(uint4* p, const uint4& v, bool nt) {
  if (nt) {
    store16_nt(p, v);
  } else {
    // one 16-B store (an ext-vector store keeps the four words together)
    const u32x4_nt r = {v.x, v.y, v.z, v.w};
    *reinterpret_cast<u32x4_nt*>(p) = r;
  }
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

// Span probes: SPAN_NT-thread workgroups, workgroup w streams the contiguous
// chunks [w * per, (w + 1) * per), SPAN_UNROLL accesses in flight per thread.
// KIND 3: read src; 4: write dst; 5: copy src -> dst; 6: update dst in place;
// 7: the momentum pack's pattern: per gradient chunk i (src[i], i < n16 / 2),
// momentum chunks 2i, 2i+1 of dst read and rewritten and X chunk n16/2 + i of
// src written (three streams of 16-B accesses, 3 x 16 x n16 bytes in all).
constexpr int SPAN_NT = 1024;
constexpr int SPAN_UNROLL = 8;
template <int KIND, bool NTA>
__global__ __launch_bounds__(SPAN_NT) void span_probe_kernel(uint4* __restrict__ dst, uint4* __restrict__ src,
                                                             int64_t n16, int64_t per) {
  const uint4 key = make_uint4(0x9E3779B9u, 0x7F4A7C15u, 0xBF58476Du, 0x1CE4E5B9u);
  if constexpr (KIND == 7) {
    // PACK_UNROLL gradient units (three loads each) in flight per thread
    constexpr int PACK_UNROLL = 2;
    const int64_t ng = n16 / 2;
    const int64_t b0 = int64_t(blockIdx.x) * per, b1 = min(ng, b0 + per);
    int64_t i = b0 + threadIdx.x;
    // every word of the three written units changes (a unit stored back
    // unchanged could be dropped by the compiler)
    auto one = [&](int64_t k, const uint4& gv, uint4 m0, uint4 m1) {
      m0.x ^= gv.x; m0.y += gv.y; m0.z ^= gv.z; m0.w += gv.w;
      m1.x += gv.x; m1.y ^= gv.y; m1.z += gv.z; m1.w ^= gv.w;
      st16(dst + 2 * k, m0, NTA);
      st16(dst + 2 * k + 1, m1, NTA);
      st16(src + ng + k, make_uint4(m0.x ^ m1.x, m0.y ^ m1.y, m0.z ^ m1.z, m0.w ^ m1.w), NTA);
    };
    for (; i + (PACK_UNROLL - 1) * SPAN_NT < b1; i += PACK_UNROLL * SPAN_NT) {
      uint4 gv[PACK_UNROLL], m0[PACK_UNROLL], m1[PACK_UNROLL];
#pragma unroll
      for (int u = 0; u < PACK_UNROLL; ++u) {
        const int64_t k = i + u * SPAN_NT;
        gv[u] = ld16(src + k, NTA);
        m0[u] = ld16(dst + 2 * k, NTA);
        m1[u] = ld16(dst + 2 * k + 1, NTA);
      }
#pragma unroll
      for (int u = 0; u < PACK_UNROLL; ++u) one(i + u * SPAN_NT, gv[u], m0[u], m1[u]);
    }
    for (; i < b1; i += SPAN_NT) one(i, ld16(src + i, NTA), ld16(dst + 2 * i, NTA), ld16(dst + 2 * i + 1, NTA));
    return;
  }
  const int64_t b0 = int64_t(blockIdx.x) * per, b1 = min(n16, b0 + per);
  int64_t i = b0 + threadIdx.x;
  uint4 acc = make_uint4(0, 0, 0, 0);
  for (; i + (SPAN_UNROLL - 1) * SPAN_NT < b1; i += SPAN_UNROLL * SPAN_NT) {
    uint4 v[SPAN_UNROLL];
#pragma unroll
    for (int u = 0; u < SPAN_UNROLL; ++u) {
      if constexpr (KIND == 4) v[u] = pattern(i + u * SPAN_NT);
      else if constexpr (KIND == 6) v[u] = ld16(dst + i + u * SPAN_NT, NTA);
      else v[u] = ld16(src + i + u * SPAN_NT, NTA);
    }
#pragma unroll
    for (int u = 0; u < SPAN_UNROLL; ++u) {
      if constexpr (KIND == 3) {
        acc.x ^= v[u].x; acc.y += v[u].y; acc.z ^= v[u].z; acc.w += v[u].w;
      } else if constexpr (KIND == 6) {
        st16(dst + i + u * SPAN_NT, make_uint4(v[u].x ^ key.x, v[u].y ^ key.y, v[u].z ^ key.z, v[u].w ^ key.w), NTA);
      } else {
        st16(dst + i + u * SPAN_NT, v[u], NTA);
      }
    }
  }
  for (; i < b1; i += SPAN_NT) {
    if constexpr (KIND == 3) {
      const uint4 v = ld16(src + i, NTA);
      acc.x ^= v.x; acc.y += v.y; acc.z ^= v.z; acc.w += v.w;
    } else if constexpr (KIND == 4) {
      st16(dst + i, pattern(i), NTA);
    } else if constexpr (KIND == 6) {
      const uint4 v = ld16(dst + i, NTA);
      st16(dst + i, make_uint4(v.x ^ key.x, v.y ^ key.y, v.z ^ key.z, v.w ^ key.w), NTA);
    } else {
      st16(dst + i, ld16(src + i, NTA), NTA);
    }
  }
  if constexpr (KIND == 3) {
    if (acc.x == key.x && acc.y == key.y && acc.z == key.z && acc.w == key.w && dst)
      dst[int64_t(blockIdx.x) * SPAN_NT + threadIdx.x] = acc;
  }
}

template <int KIND>
void launch_span(uint4* dst, uint4* src, int64_t n16, bool nt, int grid, hipStream_t s) {
  const int64_t units = KIND == 7 ? n16 / 2 : n16;
  const int64_t per = (units + grid - 1) / grid;
  if (nt) hipLaunchKernelGGL((span_probe_kernel<KIND, true>), dim3(grid), dim3(SPAN_NT), 0, s, dst, src, n16, per);
  else hipLaunchKernelGGL((span_probe_kernel<KIND, false>), dim3(grid), dim3(SPAN_NT), 0, s, dst, src, n16, per);
}

}  // namespace
}  // namespace mmuon

// Streams `bytes`-long buffers with 16-B vector accesses; nontemporal != 0 uses
// non-temporal loads and stores.
//   kind 0 / 1 / 2: read src / write dst (hashed random-looking data) / copy
//     src -> dst; grid x 256 threads, grid-stride, 4 accesses in flight;
//   kind 3 / 4 / 5 / 6: read / write / copy / update dst in place; grid x 1024
//     threads, workgroup w streams the w-th of grid contiguous spans, 8
//     accesses in flight;
//   kind 7: the momentum pack's three streams over spans: per 16-B gradient
//     unit read from src's first half, two 16-B momentum units of dst read and
//     rewritten and one 16-B unit written to src's second half (3 x bytes
//     moved), two gradient units in flight per thread.
// bytes a positive multiple of 32, buffers 16-B aligned; the read probes may
// pass dst = NULL (else dst holds grid * 4096 (kind 0) or grid * 16384 (kind 3)
// bytes).  Returns 0 or a negative MMUON_E* code (message: probe_last_error).
extern "C" const char* probe_last_error(void) { return mmuon::g_probe_err.c_str(); }

extern "C" int probe_hbm_stream(int32_t kind, void* dst, void* src, int64_t bytes, int32_t nontemporal,
                                int32_t grid, void* stream) {
  using namespace mmuon;
  char msg[160];
  if (kind < 0 || kind > 7) return set_error(MMUON_EINVAL, "kind must be in [0, 7]");
  if (bytes <= 0 || bytes % 32) return set_error(MMUON_EINVAL, "bytes must be a positive multiple of 32");
  if (grid < 1 || grid > (1 << 20)) return set_error(MMUON_EINVAL, "grid must be in [1, 2^20]");
  const bool reads_src = kind == 0 || kind == 2 || kind == 3 || kind == 5 || kind == 7;
  const bool needs_dst = kind != 0 && kind != 3;
  if ((reads_src && src == nullptr) || (needs_dst && dst == nullptr)) return set_error(MMUON_EINVAL, "null buffer");
  if ((reinterpret_cast<uintptr_t>(dst) | reinterpret_cast<uintptr_t>(src)) % 16)
    return set_error(MMUON_EINVAL, "buffers must be 16-B aligned");
  // the read probe's improbable store lands in dst[0 .. grid * 256) when dst is given
  const int64_t wg_threads = kind <= 2 ? SP_NT : SPAN_NT;
  if ((kind == 0 || kind == 3) && dst != nullptr && int64_t(grid) * wg_threads * 16 > bytes) {
    snprintf(msg, sizeof msg, "read probe: dst must hold grid * %lld bytes (%lld)", (long long)wg_threads * 16,
             (long long)grid * wg_threads * 16);
    return set_error(MMUON_EINVAL, msg);
  }
  const int64_t n16 = bytes / 16;
  auto* d = static_cast<uint4*>(dst);
  const auto* sr = static_cast<const uint4*>(src);
  auto* sw = static_cast<uint4*>(src);  // kind 7 writes its X stream into src's second half
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const bool nt = nontemporal != 0;
  switch (kind) {
    case 0: launch_probe<0>(d, sr, n16, nt, grid, s); break;
    case 1: launch_probe<1>(d, sr, n16, nt, grid, s); break;
    case 2: launch_probe<2>(d, sr, n16, nt, grid, s); break;
    case 3: launch_span<3>(d, sw, n16, nt, grid, s); break;
    case 4: launch_span<4>(d, sw, n16, nt, grid, s); break;
    case 5: launch_span<5>(d, sw, n16, nt, grid, s); break;
    case 6: launch_span<6>(d, sw, n16, nt, grid, s); break;
    default: launch_span<7>(d, sw, n16, nt, grid, s); break;
  }
  return launch_status("probe_hbm_stream");
}
