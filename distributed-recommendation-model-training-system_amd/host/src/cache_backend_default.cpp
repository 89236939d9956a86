// cache_backend_default.cpp -- the interface's default ApplyCompact.
//
// Reference: src/cache/host_backend.cpp:12-16 (the default expands the packet
// on the host and applies it as ApplyHost).  Part of the standalone library
// only; a build beside the reference links the reference's own definition
// instead of this file.
#include <future>
#include <new>
#include <utility>

#include "eps/cache_backend.hpp"
#include "job_queue.hpp"
#include "packet.hpp"

namespace eps {

std::future<Result<Ack>> CacheBackend::ApplyCompact(UpdateContext context, CompactGradients packet) {
  std::promise<Result<Ack>> refused;
  try {
    return ApplyHost(std::move(context), hipbk::ExpandPacket(packet));
  } catch (const hipbk::Fault& f) {
    refused.set_value(f.error);
  } catch (const std::bad_alloc&) {
    refused.set_value(Error{Error::Code::capacity_exceeded, "compact packet expansion ran out of memory"});
  }
  return refused.get_future();
}

}  // namespace eps
