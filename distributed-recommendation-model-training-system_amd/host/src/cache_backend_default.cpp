// cache_backend_default.cpp -- the interface's default ApplyCompact.
//
// Reference: src/cache/host_backend.cpp:12-16.  Part of the standalone
// library only; a build beside the reference links the reference's own
// definition instead of this file.
#include <future>
#include <new>
#include <utility>

#include "eps/cache_backend.hpp"
#include "executor.hpp"

namespace eps {

// Expands the CSR on the host and applies it as ApplyHost.
std::future<Result<Ack>> CacheBackend::ApplyCompact(UpdateContext context, CompactGradients packet) {
  try {
    return ApplyHost(std::move(context), hip_detail::ExpandCompact(packet));
  } catch (const hip_detail::Failure& f) {
    std::promise<Result<Ack>> p;
    p.set_value(f.error());
    return p.get_future();
  } catch (const std::bad_alloc&) {
    std::promise<Result<Ack>> p;
    p.set_value(Error{Error::Code::capacity_exceeded, "compact gradient allocation failed"});
    return p.get_future();
  }
}

}  // namespace eps
