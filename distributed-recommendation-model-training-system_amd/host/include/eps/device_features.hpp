// eps/device_features.hpp -- request of the device feature assembly.
//
// Source-compatible restatement of include/eps/device_features.hpp:5-26 of
// the reference: host partial sums, device contributions (optionally scattered
// to sequence positions) and the layouts whose mean pooling divides once.
#pragma once

#include "eps/cache_agent.hpp"

namespace eps {

struct DeviceContribution {
  DeviceTensorBlock block;
  std::vector<std::uint64_t> positions;  // projected sequence row -> compact occurrence
  bool projected = false;
};

struct SequenceProjection {
  std::uint32_t feature;
  std::uint64_t rows;
  std::vector<std::uint64_t> positions;  // compact occurrence -> sequence position
};

struct DeviceAssemblyRequest {
  std::vector<TensorBlock> host;
  std::vector<DeviceContribution> device;
  std::vector<FeatureInput> layouts;
  std::vector<SequenceProjection> projections;
};

}  // namespace eps
