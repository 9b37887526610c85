// Streaming-read probe: the practical floor of reading a given number of bytes from HBM in one
// launch on this part (launch, ramp and tail included), against which the expert kernels'
// small-batch launches are judged. Measurement only; no counterpart in the reference.
#include "../../include/specmoe_mi355x.h"
#include "smx_common.h"

namespace smx {

constexpr int kProbeThreads = 256;
constexpr int kProbeDepth = 4;  // 16-byte loads in flight per lane

// Workgroup b reads its contiguous range [b * per_wg, (b + 1) * per_wg) with non-temporal
// 16-byte loads, kProbeDepth per lane in flight; the XOR of what it read is written to sink
// only if it equals a marker, so the loads cannot be dropped and nothing is normally written.
__global__ __launch_bounds__(kProbeThreads) void stream_read_kernel(const u32x4* __restrict__ src,
                                                                    int64_t per_wg16,
                                                                    uint32_t* __restrict__ sink) {
  const u32x4* p = src + static_cast<int64_t>(blockIdx.x) * per_wg16;
  uint32_t acc = 0;
  for (int64_t i = threadIdx.x; i < per_wg16; i += kProbeThreads * kProbeDepth) {
    u32x4 v[kProbeDepth];
#pragma unroll
    for (int d = 0; d < kProbeDepth; ++d) v[d] = __builtin_nontemporal_load(p + i + d * kProbeThreads);
#pragma unroll
    for (int d = 0; d < kProbeDepth; ++d) acc ^= v[d][0] ^ v[d][1] ^ v[d][2] ^ v[d][3];
  }
  if (acc == 0x9E3779B9u) sink[0] = acc;
}

}  // namespace smx

extern "C" int smx_stream_read(const void* src, size_t bytes, size_t bytes_per_workgroup, void* sink,
                               void* stream) {
  constexpr size_t kUnit = static_cast<size_t>(smx::kProbeThreads) * 16 * smx::kProbeDepth;
  if (src == nullptr || sink == nullptr || bytes == 0 || bytes_per_workgroup == 0) return SMX_ERR_INVALID_ARG;
  if ((reinterpret_cast<uintptr_t>(src) & 15u) != 0 || (reinterpret_cast<uintptr_t>(sink) & 3u) != 0)
    return SMX_ERR_MISALIGNED;
  if (bytes_per_workgroup % kUnit != 0 || bytes % bytes_per_workgroup != 0) return SMX_ERR_INVALID_ARG;
  const size_t wgs = bytes / bytes_per_workgroup;
  if (wgs > (size_t{1} << 31) - 1) return SMX_ERR_UNSUPPORTED;
  smx::stream_read_kernel<<<static_cast<unsigned>(wgs), smx::kProbeThreads, 0,
                            static_cast<hipStream_t>(stream)>>>(
      static_cast<const smx::u32x4*>(src), static_cast<int64_t>(bytes_per_workgroup / 16),
      static_cast<uint32_t*>(sink));
  return static_cast<int>(hipGetLastError());
}
