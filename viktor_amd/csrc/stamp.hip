// Device timestamps for timing kernels inside a captured HIP graph, where events cannot be recorded between
// two nodes: a one-thread kernel stores the GPU's constant-rate wall clock (wall_clock64, read in the kernel as
// it runs) to stamps[index] with an ordinary vector store. Put one before and one after the node to time, and a
// back-to-back pair elsewhere in the same graph for the dispatch gap between two nodes; the rate comes from
// vk_timestamp_rate_khz.
#include "common.h"

namespace vk {

__global__ __launch_bounds__(64) void stamp_kernel(uint64_t *__restrict__ stamps, int64_t index) {
  if (threadIdx.x == 0) stamps[index] = static_cast<uint64_t>(wall_clock64());
}

}  // namespace vk

using namespace vk;

extern "C" int vk_timestamp(uint64_t *stamps, int64_t index, void *stream) {
  VK_CHECK_ARG(stamps && index >= 0, "timestamp: null buffer or negative index");
  stamp_kernel<<<1, 64, 0, VK_STREAM(stream)>>>(stamps, index);
  return launch_status("timestamp");
}

extern "C" int vk_timestamp_rate_khz(int64_t *khz) {
  VK_CHECK_ARG(khz, "timestamp_rate_khz: null pointer");
  int dev = 0, rate = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&rate, hipDeviceAttributeWallClockRate, dev) != hipSuccess || rate <= 0)
    return fail(VK_ERR_LAUNCH, "timestamp_rate_khz: the device reports no wall-clock rate");
  *khz = rate;
  return VK_OK;
}
