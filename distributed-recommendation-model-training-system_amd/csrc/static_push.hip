// static_push.hip -- a device push that allocates nothing.
//
// For callers that cannot allocate device memory (code under HIP graph
// capture, tight serving loops): eps_hip_prepare + eps_hip_push with the push
// workspace in a static device array of this library instead of a caller's
// buffer.  Each GPU holds its own copy of the array (from the library's load
// until the process ends) at its own address, found once per device with
// hipGetSymbolAddress; kernels get that address, never the symbol.  Calls on
// one GPU share the array, so calls that overlap on one GPU race; each call's
// preparation clears what must start at zero (with a fill kernel).  Every
// kernel of a call runs on the caller's stream (no side stream or event), and
// the only runtime calls besides launches are the first call's symbol lookup
// per device, so a call can be captured in a graph once that lookup is done.
#include <mutex>

#include "prepare.hpp"

namespace {
constexpr uint64_t kStaticBytes = eps_hip::PushLayout(EPS_HIP_STATIC_MAX_OCCURRENCES).total;
}  // namespace

// The static push workspace (zero at load, so its status history starts clean).
static __device__ __align__(256) unsigned char scratch[kStaticBytes];

namespace eps_hip {
namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch[kMaxDevices] = {};

// The current device's address of `scratch`.
int ScratchAddress(void** out) {
  int device = 0;
  EPS_HIP_TRY(Check(hipGetDevice(&device), "hipGetDevice"));
  if (device < 0 || device >= kMaxDevices) return Fail(EPS_HIP_UNAVAILABLE, "device ordinal out of range");
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch[device]) {
    void* ptr = nullptr;
    EPS_HIP_TRY(Check(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)), "hipGetSymbolAddress"));
    if (!ptr) return Fail(EPS_HIP_RUN_FAILED, "static push workspace has no device address");
    g_scratch[device] = ptr;
  }
  *out = g_scratch[device];
  return EPS_HIP_OK;
}

}  // namespace
}  // namespace eps_hip

using namespace eps_hip;

namespace eps_hip {
namespace {
// Copies a finished push's status and the static workspace's history (the
// failure bits of every static push since the last report) to the caller,
// then clears the history.
__global__ void ReportKernel(Control* ctrl, uint32_t* out) {
  out[0] = ctrl->status;
  out[1] = ctrl->history;
  ctrl->history = 0;
}
}  // namespace
}  // namespace eps_hip

extern "C" {

int eps_hip_push_static(const eps_hip_table* tables, const eps_hip_optimizer* optimizers, uint32_t table_count,
                        const eps_hip_push_feature* features, uint32_t feature_count, void* bounds,
                        uint32_t* status, void* stream) {
  if (!features && feature_count) return Fail(EPS_HIP_INVALID_ARGUMENT, "null push features");
  uint64_t occurrences = 0;
  for (uint32_t f = 0; f < feature_count; ++f) occurrences += features[f].occurrences;
  if (occurrences > EPS_HIP_STATIC_MAX_OCCURRENCES)
    return Fail(EPS_HIP_CAPACITY_EXCEEDED, "a static push holds at most 262144 occurrences "
                                           "(EPS_HIP_STATIC_MAX_OCCURRENCES); larger pushes take "
                                           "eps_hip_prepare + eps_hip_push with a workspace");
  void* ws = nullptr;
  EPS_HIP_TRY(ScratchAddress(&ws));
  EPS_HIP_TRY(eps_hip_prepare(tables, table_count, features, feature_count, ws, kStaticBytes, stream));
  EPS_HIP_TRY(PushOneStream(tables, optimizers, table_count, features, feature_count, ws, kStaticBytes, bounds,
                            stream));
  if (status) {
    hipLaunchKernelGGL(ReportKernel, dim3(1), dim3(1), 0, AsStream(stream), static_cast<Control*>(ws), status);
    EPS_HIP_LAUNCHED("static push status");
  }
  return EPS_HIP_OK;
}

}  // extern "C"
