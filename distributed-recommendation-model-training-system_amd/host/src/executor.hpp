// executor.hpp -- the backend's single FIFO worker and its error conventions.
//
// Same contract as the reference's OrderedExecutor and Failure/Require
// (src/common/executor.hpp:12-50, src/common/error.hpp:10-22): jobs run one at
// a time in submission order on one thread, each resolves a future<Result<T>>,
// a full queue resolves immediately to capacity_exceeded, and exceptions never
// cross the interface (Failure -> its Error, bad_alloc -> capacity_exceeded,
// anything else -> run_failed).  Private namespace: links beside the
// reference's own eps::detail.
#pragma once

#include <condition_variable>
#include <deque>
#include <functional>
#include <future>
#include <memory>
#include <mutex>
#include <stdexcept>
#include <string>
#include <thread>

#include "eps/types.hpp"

namespace eps::hip_detail {

class Failure : public std::runtime_error {
 public:
  explicit Failure(Error error) : std::runtime_error(error.message), error_(std::move(error)) {}
  const Error& error() const { return error_; }

 private:
  Error error_;
};

inline void Require(bool condition, const char* message,
                    Error::Code code = Error::Code::invalid_argument) {
  if (!condition) throw Failure({code, message});
}

class Worker {
 public:
  explicit Worker(std::size_t max_jobs) : limit_(max_jobs), thread_([this] { Run(); }) {}
  ~Worker() { Stop(); }
  Worker(const Worker&) = delete;
  Worker& operator=(const Worker&) = delete;

  // Drains queued jobs and joins; idempotent.  Owners call it before the state
  // that queued jobs refer to is destroyed.
  void Stop() {
    std::call_once(stopped_, [this] {
      {
        std::lock_guard<std::mutex> lock(mutex_);
        stopping_ = true;
      }
      wake_.notify_all();
      thread_.join();
    });
  }

  template <typename T, typename F>
  std::future<Result<T>> Submit(F fn) {
    auto promise = std::make_shared<std::promise<Result<T>>>();
    auto future = promise->get_future();
    {
      std::lock_guard<std::mutex> lock(mutex_);
      if (stopping_ || jobs_.size() >= limit_) {
        promise->set_value(Error{Error::Code::capacity_exceeded, "agent queue is full"});
        return future;
      }
      jobs_.emplace_back([promise, fn = std::move(fn)]() mutable {
        try {
          promise->set_value(fn());
        } catch (const Failure& f) {
          promise->set_value(f.error());
        } catch (const std::bad_alloc&) {
          promise->set_value(Error{Error::Code::capacity_exceeded, "agent allocation failed"});
        } catch (const std::exception& e) {
          promise->set_value(Error{Error::Code::run_failed, e.what()});
        }
      });
    }
    wake_.notify_one();
    return future;
  }

 private:
  void Run() {
    for (;;) {
      std::function<void()> job;
      {
        std::unique_lock<std::mutex> lock(mutex_);
        wake_.wait(lock, [this] { return stopping_ || !jobs_.empty(); });
        if (jobs_.empty()) return;  // stopping and drained
        job = std::move(jobs_.front());
        jobs_.pop_front();
      }
      job();
    }
  }

  std::size_t limit_;
  std::mutex mutex_;
  std::condition_variable wake_;
  std::deque<std::function<void()>> jobs_;
  bool stopping_ = false;
  std::once_flag stopped_;
  std::thread thread_;
};

// CSR packet checks and host expansion (reference:
// src/access/compact_gradients.cpp:10-39): the whole packet is validated before
// any state changes; expansion sums src*scale per reference in order.
void ValidateCompact(const CompactGradients& packet);
std::uint64_t CompactBytes(const CompactGradients& packet);
RowGradients ExpandCompact(const CompactGradients& packet);

}  // namespace eps::hip_detail
