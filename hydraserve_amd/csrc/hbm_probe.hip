// Streaming-read probe: the HBM read ceiling of this part, measured with the
// simplest access pattern (every byte of a buffer read once, 16-byte loads,
// consecutive lanes on consecutive addresses, many loads in flight per lane).
// The decode GEMMs are priced against 8 TB/s; this kernel states what a read
// with no compute reaches, so their roofline fraction can be read against a
// measured ceiling as well as the nominal one.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "../../include/hydraserve_amd.h"

namespace hsq {
namespace {

constexpr int kProbeThreads = 256;
constexpr int kProbeUnroll = 8;

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(kProbeThreads) void hbm_read_probe_kernel(const u32x4_t* __restrict__ src,
                                                                       int64_t n16, uint32_t* __restrict__ sink) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kProbeThreads;
  int64_t i = static_cast<int64_t>(blockIdx.x) * kProbeThreads + threadIdx.x;
  u32x4_t acc = {0u, 0u, 0u, 0u};
  for (; i + (kProbeUnroll - 1) * stride < n16; i += kProbeUnroll * stride) {
    u32x4_t v[kProbeUnroll];
#pragma unroll
    for (int u = 0; u < kProbeUnroll; ++u) v[u] = __builtin_nontemporal_load(src + i + u * stride);
#pragma unroll
    for (int u = 0; u < kProbeUnroll; ++u) acc ^= v[u];
  }
  for (; i < n16; i += stride) acc ^= src[i];
  const uint32_t r = acc.x ^ acc.y ^ acc.z ^ acc.w;
  // Lane 0 stores its value; every other lane's value feeds a store the
  // compiler cannot rule out (it happens only for one 32-bit value), so no
  // lane's loads can be dropped while only one word per workgroup is written.
  if (threadIdx.x == 0) sink[blockIdx.x] = r;
  else if (r == 0x9e3779b9u) sink[blockIdx.x] = r + threadIdx.x;
}

}  // namespace
}  // namespace hsq

extern "C" int hs_hbm_read_probe(const void* src, int64_t bytes, void* sink, int64_t sink_bytes, int blocks,
                                 void* stream) {
  if (src == nullptr || sink == nullptr || bytes < 16 || (bytes & 15) != 0 || blocks <= 0 ||
      (reinterpret_cast<uintptr_t>(src) & 15) != 0)
    return HS_EINVAL;
  if (sink_bytes < static_cast<int64_t>(blocks) * 4) return HS_EINVAL;
  hipLaunchKernelGGL(hsq::hbm_read_probe_kernel, dim3(blocks), dim3(hsq::kProbeThreads), 0,
                     static_cast<hipStream_t>(stream), static_cast<const hsq::u32x4_t*>(src), bytes / 16,
                     static_cast<uint32_t*>(sink));
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? HS_OK : HS_EHIP + static_cast<int>(e);
}
