// Streaming-read probe: the HBM read rate this GPU sustains for a given byte count, as the
// ceiling the decode kernels are compared against.  It reads `bytes` once with
// non-temporal 16-byte loads (the access the decode kernels make for cache codes) and
// folds them with XOR, so the loads cannot be dropped; one word per work-group is stored
// only when the fold hits a fixed 32-bit value (practically never), so it writes nothing.
//
// Work-group g reads the g-th of work_groups contiguous slabs front to back, 8 loads of
// 16 bytes in flight per lane.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>

#include "kvq.h"

namespace kvq {

extern thread_local std::string g_last_error;
int fail(int code, const std::string& msg);

namespace {

constexpr int kProbeThreads = 512;
constexpr int kProbeUnroll = 8;
constexpr uint32_t kProbeMagic = 0x9E3779B9u;
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(kProbeThreads) void stream_read_kernel(const u32x4_t* __restrict__ p,
                                                                     uint64_t n16,
                                                                     uint32_t* __restrict__ sink) {
  // work-group g streams the contiguous units [g * per, (g + 1) * per) front to back, 8 KiB
  // per load instruction of the work-group and kProbeUnroll of them in flight
  const uint64_t per = (n16 + gridDim.x - 1) / gridDim.x;
  const uint64_t lo = (uint64_t)blockIdx.x * per;
  const uint64_t hi = lo + per < n16 ? lo + per : n16;
  constexpr uint64_t kStep = (uint64_t)kProbeThreads * kProbeUnroll;
  uint64_t i = lo + threadIdx.x;
  uint32_t acc = 0;
  for (; i + (kProbeUnroll - 1) * kProbeThreads < hi; i += kStep) {
    u32x4_t v[kProbeUnroll];
#pragma unroll
    for (int u = 0; u < kProbeUnroll; ++u) v[u] = __builtin_nontemporal_load(p + i + u * kProbeThreads);
#pragma unroll
    for (int u = 0; u < kProbeUnroll; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  for (; i < hi; i += kProbeThreads) {
    const u32x4_t v = __builtin_nontemporal_load(p + i);
    acc ^= v.x ^ v.y ^ v.z ^ v.w;
  }
  if (acc == kProbeMagic) sink[blockIdx.x] = acc;
}

}  // namespace
}  // namespace kvq

extern "C" int kvq_stream_read(const void* buf, int64_t bytes, uint32_t* sink, int32_t work_groups,
                               kvq_stream_t stream) {
  using namespace kvq;
  if (!buf || !sink) return fail(KVQ_ERR_INVALID, "stream_read: buf / sink is NULL");
  if (bytes <= 0 || bytes % 16) return fail(KVQ_ERR_INVALID, "stream_read: bytes must be a positive multiple of 16");
  if (((uintptr_t)buf) % 16) return fail(KVQ_ERR_INVALID, "stream_read: buf must be 16-byte aligned");
  if (work_groups <= 0 || work_groups > (1 << 20))
    return fail(KVQ_ERR_INVALID, "stream_read: work_groups must be in [1, 2^20]");
  hipLaunchKernelGGL(stream_read_kernel, dim3((unsigned)work_groups), dim3(kProbeThreads), 0,
                     reinterpret_cast<hipStream_t>(stream), reinterpret_cast<const u32x4_t*>(buf),
                     (uint64_t)bytes / 16, sink);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(KVQ_ERR_LAUNCH, std::string("launch: ") + hipGetErrorString(e));
  return KVQ_OK;
}
