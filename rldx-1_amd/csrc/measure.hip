// HBM read-rate probe for the benchmark's measured ceilings (bench.py
// `measured_peaks.read_gbs`): the rate at which this GPU streams bytes from
// device memory into registers, with nothing else in the kernel.  A library
// reduction (torch.sum) reaches only ~3.5 TB/s on MI355X, well below what a
// streaming kernel gets, so a kernel line's "fraction of the measured read"
// uses this probe instead.
//
// Design: 256 workgroups of 256 threads (one per CU), a grid-stride loop of
// 16-byte loads with 8 independent loads per thread in flight (32 KB per CU),
// results folded with XOR; the only store is taken when the fold equals a
// constant, so the loads stay live and the kernel writes (almost) nothing.
// Measured on MI355X over 3 rotated 512 MiB buffers: 6.5 TB/s; the same loop
// over 1024-4096 workgroups reads 4.7-5.6 TB/s, a workgroup-contiguous
// (blocked) split 5.8-6.3 TB/s.
#include "rldx_amd.h"
#include "rldx_common.h"

namespace rldx {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kProbeThreads = 256;
constexpr int kProbeUnroll = 8;

__global__ __launch_bounds__(kProbeThreads) void read_probe_kernel(const u32x4* __restrict__ p, int64_t n16,
                                                                   uint32_t* __restrict__ sink) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kProbeThreads;
  int64_t i = static_cast<int64_t>(blockIdx.x) * kProbeThreads + threadIdx.x;
  u32x4 acc = {0u, 0u, 0u, 0u};
  for (; i + (kProbeUnroll - 1) * stride < n16; i += kProbeUnroll * stride) {
    u32x4 v[kProbeUnroll];
#pragma unroll
    for (int u = 0; u < kProbeUnroll; ++u) v[u] = p[i + u * stride];
#pragma unroll
    for (int u = 0; u < kProbeUnroll; ++u) acc ^= v[u];
  }
  for (; i < n16; i += stride) acc ^= p[i];
  const uint32_t f = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
  if (f == 0x9e3779b9u) sink[blockIdx.x] = f;
}

}  // namespace
}  // namespace rldx

extern "C" int64_t rldx_read_probe_sink_words(void) { return 256; }

extern "C" hipError_t rldx_read_probe(const void* data, int64_t bytes, void* sink, int64_t sink_words,
                                      hipStream_t stream) {
  if (bytes < 0 || bytes % 16 || sink_words < rldx_read_probe_sink_words()) return hipErrorInvalidValue;
  if (bytes == 0) return hipSuccess;
  if (!data || !sink || reinterpret_cast<uintptr_t>(data) % 16 || reinterpret_cast<uintptr_t>(sink) % 4)
    return hipErrorInvalidValue;
  hipLaunchKernelGGL(rldx::read_probe_kernel, dim3(static_cast<unsigned>(rldx_read_probe_sink_words())),
                     dim3(rldx::kProbeThreads), 0, stream, static_cast<const rldx::u32x4*>(data), bytes / 16,
                     static_cast<uint32_t*>(sink));
  return hipGetLastError();
}
