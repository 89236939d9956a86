// eps/cache_agent.hpp -- device-resident results of a GPU cache agent.
//
// Source-compatible restatement of include/eps/cache_agent.hpp:7-23 of the
// reference.  WaitOnStream takes the consumer's stream (a hipStream_t here).
#pragma once

#include "eps/cache_backend.hpp"

namespace eps {

struct DeviceTensor {
  virtual ~DeviceTensor() = default;
  virtual void* data() const = 0;
  virtual std::uint64_t elements() const = 0;
  virtual int device() const = 0;
  virtual void WaitOnStream(void* stream) const = 0;
  virtual std::vector<float> CopyToHost() const = 0;
};

class GpuCacheAgent : public CacheBackend {
 public:
  virtual std::future<Result<std::vector<DeviceTensorBlock>>> GatherDevice(
      std::vector<AgentWork> work, std::vector<FeatureInput> layouts) = 0;
};

}  // namespace eps
