// job_queue_test.cpp -- host unit test of the backend's operation queue
// (host/src/job_queue.hpp), no GPU.
//
// The contract it keeps from the reference (src/common/executor.hpp:11-50,
// src/cuda/cache_backend.cu:222): operations run one at a time in submission
// order on one thread; at most `depth` wait, and a call beyond that resolves at
// once to capacity_exceeded without running; a job's Fault becomes its error,
// std::bad_alloc capacity_exceeded and any other exception run_failed; Close
// runs what is queued and refuses what comes after.
#include <chrono>
#include <cstdio>
#include <future>
#include <new>
#include <stdexcept>
#include <string>
#include <vector>

#include "job_queue.hpp"

using namespace eps;
using eps::hipbk::JobQueue;

namespace {

int failures = 0;
void Expect(bool ok, const char* what) {
  if (!ok) {
    std::fprintf(stderr, "FAIL: %s\n", what);
    ++failures;
  }
}

template <typename T>
bool Refused(std::future<Result<T>>& f, Error::Code code) {
  auto r = f.get();
  return std::holds_alternative<Error>(r) && std::get<Error>(r).code == code;
}

void DepthAndOrder() {
  constexpr std::size_t kDepth = 128;
  JobQueue queue(kDepth);
  std::promise<void> started, gate;
  std::shared_future<void> open = gate.get_future().share();
  // The first job holds the worker until the gate opens; wait until it runs,
  // so the queue is empty and exactly kDepth more can wait.
  auto blocker = queue.Post<int>([&] {
    started.set_value();
    open.wait();
    return -1;
  });
  started.get_future().wait();
  std::vector<int> order;
  std::vector<std::future<Result<int>>> waiting;
  for (std::size_t i = 0; i < kDepth; ++i)
    waiting.push_back(queue.Post<int>([&order, i] {
      order.push_back(int(i));
      return int(i);
    }));
  bool ran_refused = false;
  auto refused = queue.Post<int>([&] {
    ran_refused = true;
    return 0;
  });
  Expect(refused.wait_for(std::chrono::seconds(0)) == std::future_status::ready,
         "a call beyond the depth resolves at once");
  Expect(Refused(refused, Error::Code::capacity_exceeded), "a call beyond the depth is capacity_exceeded");
  gate.set_value();
  Expect(std::get<int>(blocker.get()) == -1, "blocking job result");
  for (std::size_t i = 0; i < kDepth; ++i) Expect(std::get<int>(waiting[i].get()) == int(i), "queued job result");
  bool in_order = order.size() == kDepth;
  for (std::size_t i = 0; in_order && i < kDepth; ++i) in_order = order[i] == int(i);
  Expect(in_order, "jobs ran in submission order");
  Expect(!ran_refused, "a refused job never runs");
  // Room again once drained.
  auto after = queue.Post<int>([] { return 7; });
  Expect(std::get<int>(after.get()) == 7, "queue accepts after draining");
}

void ErrorMapping() {
  JobQueue queue(8);
  auto fault = queue.Post<int>([]() -> int { hipbk::Raise(Error::Code::stale_generation, "stale"); });
  auto alloc = queue.Post<int>([]() -> int { throw std::bad_alloc(); });
  auto other = queue.Post<int>([]() -> int { throw std::runtime_error("boom"); });
  auto check = queue.Post<int>([]() -> int {
    hipbk::Expect(false, "argument");
    return 0;
  });
  auto fine = queue.Post<int>([] { return 1; });
  Expect(Refused(fault, Error::Code::stale_generation), "a Fault keeps its code");
  Expect(Refused(alloc, Error::Code::capacity_exceeded), "bad_alloc is capacity_exceeded");
  Expect(Refused(other, Error::Code::run_failed), "another exception is run_failed");
  Expect(Refused(check, Error::Code::invalid_argument), "Expect is invalid_argument");
  Expect(std::get<int>(fine.get()) == 1, "a job after failed ones runs");
}

void CloseDrains() {
  auto queue = std::make_unique<JobQueue>(8);
  std::vector<std::future<Result<int>>> jobs;
  int ran = 0;
  for (int i = 0; i < 8; ++i)
    jobs.push_back(queue->Post<int>([&ran, i] {
      ++ran;
      return i;
    }));
  queue->Close();
  Expect(ran == 8, "Close runs every queued job");
  for (int i = 0; i < 8; ++i) Expect(std::get<int>(jobs[i].get()) == i, "queued result after Close");
  auto late = queue->Post<int>([] { return 0; });
  Expect(Refused(late, Error::Code::capacity_exceeded), "a call after Close is refused");
  queue->Close();  // idempotent
}

}  // namespace

int main() {
  DepthAndOrder();
  ErrorMapping();
  CloseDrains();
  if (failures) return 1;
  std::printf("job_queue_test: ok\n");
  return 0;
}
