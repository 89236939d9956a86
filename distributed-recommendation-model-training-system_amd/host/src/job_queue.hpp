// job_queue.hpp -- how a HipCacheBackend runs its operations and reports errors.
//
// Contract kept from the reference backend (src/common/executor.hpp:11-50,
// src/common/error.hpp): operations of one backend run one at a time, in the
// order they were submitted, on one thread; each resolves a
// future<Result<T>>; at most `depth` operations wait (then the call resolves
// at once to capacity_exceeded); no exception ever reaches the caller.
//
// Inside a job an error is thrown as a Fault (an eps::Error); allocation
// failure becomes capacity_exceeded and any other exception run_failed.
#pragma once

#include <condition_variable>
#include <deque>
#include <exception>
#include <functional>
#include <future>
#include <memory>
#include <mutex>
#include <new>
#include <string>
#include <thread>
#include <utility>

#include "eps/types.hpp"

namespace eps::hipbk {

struct Fault {
  Error error;
};

[[noreturn]] inline void Raise(Error::Code code, std::string message) {
  throw Fault{Error{code, std::move(message)}};
}
// An argument or request check (invalid_argument unless stated).
inline void Expect(bool ok, const char* message, Error::Code code = Error::Code::invalid_argument) {
  if (!ok) Raise(code, message);
}

// Resolves `promise` with fn()'s value, or with the error it raised.
template <typename T, typename F>
void Settle(std::promise<Result<T>>& promise, F& fn) {
  try {
    promise.set_value(fn());
  } catch (const Fault& f) {
    promise.set_value(f.error);
  } catch (const std::bad_alloc&) {
    promise.set_value(Error{Error::Code::capacity_exceeded, "backend host allocation failed"});
  } catch (const std::exception& e) {
    promise.set_value(Error{Error::Code::run_failed, e.what()});
  }
}

class JobQueue {
 public:
  explicit JobQueue(std::size_t depth) : depth_(depth), thread_([this] { Serve(); }) {}
  ~JobQueue() { Close(); }
  JobQueue(const JobQueue&) = delete;
  JobQueue& operator=(const JobQueue&) = delete;

  // Refuses new jobs, runs the queued ones, joins the thread.  Idempotent;
  // the owner calls it before the state the jobs use goes away.
  void Close() {
    {
      std::lock_guard<std::mutex> lock(mutex_);
      if (closed_) return;
      closed_ = true;
    }
    ready_.notify_all();
    if (thread_.joinable()) thread_.join();
  }

  template <typename T, typename F>
  std::future<Result<T>> Post(F fn) {
    auto promise = std::make_shared<std::promise<Result<T>>>();
    std::future<Result<T>> result = promise->get_future();
    bool queued = false;
    {
      std::lock_guard<std::mutex> lock(mutex_);
      if (!closed_ && pending_.size() < depth_) {
        pending_.emplace_back([promise, fn = std::move(fn)]() mutable { Settle(*promise, fn); });
        queued = true;
      }
    }
    if (queued) {
      ready_.notify_one();
    } else {
      promise->set_value(Error{Error::Code::capacity_exceeded, "backend job queue is full"});
    }
    return result;
  }

 private:
  void Serve() {
    std::unique_lock<std::mutex> lock(mutex_);
    for (;;) {
      ready_.wait(lock, [this] { return closed_ || !pending_.empty(); });
      if (pending_.empty()) return;  // closed and drained
      std::function<void()> job = std::move(pending_.front());
      pending_.pop_front();
      lock.unlock();
      job();
      lock.lock();
    }
  }

  const std::size_t depth_;
  std::mutex mutex_;
  std::condition_variable ready_;
  std::deque<std::function<void()>> pending_;
  bool closed_ = false;
  std::thread thread_;
};

}  // namespace eps::hipbk
