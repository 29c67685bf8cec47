// Stream holder of the host API, in place of the reference's
// kernel::CudaConfig (include/base/cuda_config.h:6-13): owns a HIP stream
// created through the C ABI and destroys it with the config.
#pragma once

namespace kernel {
struct HipConfig {
  void* stream = nullptr;  // hipStream_t
  HipConfig() = default;
  HipConfig(const HipConfig&) = delete;
  HipConfig& operator=(const HipConfig&) = delete;
  ~HipConfig();
  // Creates the stream (kl_stream_create); returns 0 or the C ABI's code.
  int create();
};
}  // namespace kernel
