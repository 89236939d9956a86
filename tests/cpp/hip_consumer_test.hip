// hip_consumer_test.hip -- device outputs of eps::HipCacheBackend handed to a
// model on its own stream, and the outstanding-output budget, on a GPU.
//
// The scenario of the reference's tests/worker_agent_cuda.cu:50-81, against
// the backend directly (the worker agent and its RPC control are not part of
// this library): a budget of 160 bytes, two rows of dimension 4 and a request
// of a sum feature (bags {1,1}, {2}, {}) and a sequence feature ({2, 1}),
// whose outputs take 48 + 32 = 80 bytes.
//  * a model kernel on a non-blocking stream of its own reads each output
//    after WaitOnStream(stream) and computes 2x + 1, equal bit for bit to the
//    same arithmetic on the host's sequential sums;
//  * a second request fits the budget, a third is refused with
//    capacity_exceeded, the outstanding bytes read 160, and 80 once the second
//    result is released; a request larger than the whole budget is refused;
//  * the first result outlives the backend: the model reads it again, with
//    the same answer, after the backend is destroyed.
// Prints PASS and one JSON line; any failure prints FAIL and exits 1.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstring>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "eps/hip_cache_backend.hpp"

using namespace eps;

namespace {

void Check(bool ok, const std::string& why) {
  if (!ok) throw std::runtime_error(why);
}
void HipOk(hipError_t e, const char* what) {
  if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

template <typename T>
T Take(std::future<Result<T>> f) {
  auto r = f.get();
  if (auto e = std::get_if<Error>(&r)) throw std::runtime_error("backend error: " + e->message);
  return std::get<T>(std::move(r));
}

__global__ void Model(const float* features, float* output, std::uint64_t count) {
  const std::uint64_t i = std::uint64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < count) output[i] = 2.0f * features[i] + 1.0f;
}

// A consumer with its own non-blocking stream and a 256-float output.
struct Consumer {
  hipStream_t stream = nullptr;
  float* output = nullptr;
  Consumer() {
    HipOk(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking), "consumer stream");
    HipOk(hipMalloc(&output, 256 * sizeof(float)), "consumer output");
  }
  ~Consumer() {
    if (stream) (void)hipStreamSynchronize(stream);
    if (output) (void)hipFree(output);
    if (stream) (void)hipStreamDestroy(stream);
  }
  std::vector<float> Run(const DeviceTensorBlock& input) {
    const std::uint64_t n = input.tensor->elements();
    Check(n <= 256, "consumer output bound");
    input.tensor->WaitOnStream(stream);
    if (n) {
      hipLaunchKernelGGL(Model, dim3(unsigned((n + 255) / 256)), dim3(256), 0, stream,
                         static_cast<const float*>(input.tensor->data()), output, n);
      HipOk(hipGetLastError(), "model launch");
    }
    std::vector<float> result(n);
    if (n) HipOk(hipMemcpyAsync(result.data(), output, n * 4, hipMemcpyDeviceToHost, stream), "model copy");
    HipOk(hipStreamSynchronize(stream), "model sync");
    return result;
  }
};

bool SameBits(const std::vector<float>& a, const std::vector<float>& b) {
  return a.size() == b.size() && (a.empty() || std::memcmp(a.data(), b.data(), a.size() * 4) == 0);
}

void Main() {
  HipCacheOptions options;
  options.rows_per_table = 4;
  options.state_bytes = 1 << 20;
  options.transfer_bytes = 1 << 20;
  options.outstanding_output_bytes = 160;
  auto backend = std::make_shared<HipCacheBackend>(options);
  std::weak_ptr<HipCacheBackend> lifetime = backend;
  Take(backend->Define({1, 4, 1, 1, {0.01f, 0.9f, 0.999f, 1e-8f, 0.9f, 0.999f}, 0.f, 0.f, 42}));
  const std::vector<float> w1{0.1f, 0.2f, 0.3f, 0.4f}, w2{0.5f, 0.6f, 0.7f, 0.8f};
  std::vector<RowState> initial{{{1, 1}, w1, {0, 0, 0, 0}, {0, 0, 0, 0}, 0},
                                {{1, 2}, w2, {0, 0, 0, 0}, {0, 0, 0, 0}, 0}};
  MigrationPlan load{"load", 0, {{{1, 1}, 0, Placement::loading, 0, 1, 0}, {{1, 2}, 0, Placement::loading, 0, 1, 0}},
                     Placement::gpu, 96};
  const auto rows = Take(backend->Load(load, initial));
  const std::vector<AgentWork> work{{10, AccessRoute::resident_gpu, 0, rows, {0, 0, 1}, {}},
                                    {11, AccessRoute::resident_gpu, 0, rows, {1, 0}, {}}};
  const std::vector<FeatureInput> layouts{{1, 10, Pooling::sum, {1, 1, 2}, {0, 2, 3, 3}, {2, 1, 0}},
                                          {1, 11, Pooling::sequence, {2, 1}, {0, 2}, {2}}};

  // Expected pooled values: sequential fp32 sums of each bag, then the model.
  std::vector<float> bags(12, 0.f), sequence(8);
  for (int d = 0; d < 4; ++d) {
    bags[d] = w1[d] + w1[d];
    bags[4 + d] = w2[d];
    sequence[d] = w2[d];
    sequence[4 + d] = w1[d];
  }
  auto model = [](std::vector<float> v) {
    for (auto& x : v) {
      const volatile float twice = 2.0f * x;
      x = twice + 1.0f;
    }
    return v;
  };
  const std::vector<std::vector<float>> wanted{model(bags), model(sequence)};
  const std::vector<std::vector<std::uint64_t>> shapes{{3, 4}, {2, 4}};

  Consumer consumer;
  auto first = Take(backend->GatherDevice(work, layouts));
  Check(first.size() == 2, "device result count");
  for (std::size_t f = 0; f < first.size(); ++f) {
    Check(first[f].feature == layouts[f].feature && first[f].shape == shapes[f], "device feature layout");
    Check(SameBits(consumer.Run(first[f]), wanted[f]), "model on the consumer stream, feature " + std::to_string(f));
  }

  auto second = Take(backend->GatherDevice(work, layouts));
  auto rejected = backend->GatherDevice(work, layouts).get();
  Check(std::holds_alternative<Error>(rejected) && std::get<Error>(rejected).code == Error::Code::capacity_exceeded,
        "device output budget not enforced");
  Check(Take(backend->MemoryStats()).outstanding_output_bytes == 160, "outstanding output bytes with two results");
  second.clear();
  Check(Take(backend->MemoryStats()).outstanding_output_bytes == 80, "outstanding output bytes after a release");

  // One request larger than the whole budget: 41 bags of dimension 4.
  FeatureInput wide{1, 12, Pooling::sum, {}, {0}, {}};
  AgentWork wide_work{12, AccessRoute::resident_gpu, 0, rows, {}, {}};
  for (std::uint64_t b = 0; b < 41; ++b) {
    wide.keys.push_back(1);
    wide_work.occurrence_to_unique.push_back(0);
    wide.offsets.push_back(b + 1);
    wide.valid_lengths.push_back(1);
  }
  auto too_big = backend->GatherDevice({wide_work}, {wide}).get();
  Check(std::holds_alternative<Error>(too_big) && std::get<Error>(too_big).code == Error::Code::capacity_exceeded,
        "an output larger than the budget was accepted");
  Check(Take(backend->MemoryStats()).outstanding_output_bytes == 80, "a refused request changed the budget");

  backend.reset();
  Check(lifetime.expired(), "backend not destroyed");
  for (std::size_t f = 0; f < first.size(); ++f)
    Check(SameBits(consumer.Run(first[f]), wanted[f]), "result read after the backend ended");
  first.clear();
}

}  // namespace

int main() {
  try {
    Main();
  } catch (const std::exception& e) {
    std::fprintf(stderr, "FAIL hip consumer: %s\n", e.what());
    return 1;
  }
  std::printf("PASS\n{\"test\": \"hip_consumer_stream\", \"model_stream\": \"nonblocking\", "
              "\"output_budget_enforced\": true, \"result_outlives_backend\": true}\n");
  return 0;
}
