// row_rmw.hip -- the bandwidth ceiling of the row update's access pattern.
// Measurement code only: built into libeps_hip_measure.so, which bench.py's
// ceiling run loads; the kernel library and its C ABI do not contain it.
//
// The fused update reads each touched row's [w | m | v] (3 x dim floats, at a
// random slot), reads the gradient rows that reference it, and writes the row
// back.  This kernel does exactly that traffic with a trivial update and no
// sorted-run bookkeeping, so its rate is what the memory system gives that
// pattern: the row update's roofline measured instead of assumed.  It changes
// the rows it is given (w -= 1e-3 * m and the moments move), so it runs on a
// scratch table only.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>

#include "../csrc/common.hpp"

namespace eps_hip {
namespace {

// Groups of G = dim / 4 lanes (4 columns a lane); each group updates kRows
// consecutive list entries per pass with all their loads issued first.
template <uint32_t kRows>
__global__ void __launch_bounds__(kBlock) RowRmwProbeKernel(float* state, uint32_t dim, uint32_t log2g,
                                                            const uint64_t* slots, uint64_t n,
                                                            const float* grad, uint64_t grad_rows) {
  const uint32_t G = 1u << log2g;
  const uint32_t lig = threadIdx.x & (G - 1);
  const uint64_t groups = (uint64_t(gridDim.x) * kBlock) >> log2g;
  const uint32_t c = lig * 4;
  for (uint64_t r0 = ((uint64_t(blockIdx.x) * kBlock + threadIdx.x) >> log2g) * kRows; r0 < n;
       r0 += groups * kRows) {
    float4 w[kRows], m[kRows], v[kRows], g[kRows];
    float* row[kRows];
#pragma unroll
    for (uint32_t k = 0; k < kRows; ++k) {
      const uint64_t i = min(r0 + k, n - 1);
      row[k] = state + slots[i] * dim * 3;
      // A fixed scatter of the list index over the gradient rows, as the
      // references of sorted keys land on unrelated bags.
      const uint64_t gr = (i * 0x9E3779B1ull) % grad_rows;
      w[k] = Load4Stream(row[k] + c);
      m[k] = Load4Stream(row[k] + dim + c);
      v[k] = Load4Stream(row[k] + 2 * dim + c);
      g[k] = Load4(grad + gr * dim + c);
    }
#pragma unroll
    for (uint32_t k = 0; k < kRows; ++k) {
      if (r0 + k >= n) break;
      auto step = [](float& wx, float& mx, float& vx, float gx) {
        mx = 0.9f * mx + 0.1f * gx;
        vx = 0.999f * vx + 0.001f * gx * gx;
        wx = wx - 1e-3f * mx;
      };
      step(w[k].x, m[k].x, v[k].x, g[k].x);
      step(w[k].y, m[k].y, v[k].y, g[k].y);
      step(w[k].z, m[k].z, v[k].z, g[k].z);
      step(w[k].w, m[k].w, v[k].w, g[k].w);
      Store4Stream(row[k] + c, w[k]);
      Store4Stream(row[k] + dim + c, m[k]);
      Store4Stream(row[k] + 2 * dim + c, v[k]);
    }
  }
}

}  // namespace
}  // namespace eps_hip

using namespace eps_hip;

namespace {
thread_local std::string measure_error;
int Reject(const char* message) {
  measure_error = message;
  return EPS_HIP_INVALID_ARGUMENT;
}
}  // namespace

// For list entries i < n: read row slots[i]'s [w | m | v] (3 x dim floats of
// `state`) and one gradient row (gradients + ((i * 0x9E3779B1) %
// gradient_rows) * dim), apply a fixed moment update, write the row back.
// Every slot must be < the rows `state` holds and distinct; the rows are
// changed, so `state` is a scratch table.  dim: a power of two in [4, 256];
// rows_per_group: 1, 2 or 4 entries with their loads in flight per group of
// dim/4 lanes; grid: workgroups of 256.  Returns 0 or EPS_HIP_INVALID_ARGUMENT
// / EPS_HIP_RUN_FAILED with eps_measure_last_error() saying why.
extern "C" int eps_measure_row_rmw(float* state, uint32_t dim, const uint64_t* slots, uint64_t n,
                                   const float* gradients, uint64_t gradient_rows, uint32_t rows_per_group,
                                   uint32_t grid, void* stream) {
  if (!n) return EPS_HIP_OK;
  if (!state || !slots || !gradients || !gradient_rows) return Reject("null row probe buffers");
  if (dim < 4 || dim > 256 || (dim & (dim - 1)))
    return Reject("row probe dimension must be a power of two in [4, 256]");
  if (grid == 0 || grid > 65536) return Reject("row probe grid must be in [1, 65536]");
  uint32_t log2g = 0;
  while ((4u << log2g) < dim) ++log2g;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  switch (rows_per_group) {
    case 1: hipLaunchKernelGGL(RowRmwProbeKernel<1>, dim3(grid), dim3(kBlock), 0, s, state, dim, log2g, slots, n,
                               gradients, gradient_rows); break;
    case 2: hipLaunchKernelGGL(RowRmwProbeKernel<2>, dim3(grid), dim3(kBlock), 0, s, state, dim, log2g, slots, n,
                               gradients, gradient_rows); break;
    case 4: hipLaunchKernelGGL(RowRmwProbeKernel<4>, dim3(grid), dim3(kBlock), 0, s, state, dim, log2g, slots, n,
                               gradients, gradient_rows); break;
    default: return Reject("row probe rows per group must be 1, 2 or 4");
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    measure_error = std::string("row probe launch: ") + hipGetErrorString(e);
    return EPS_HIP_RUN_FAILED;
  }
  return EPS_HIP_OK;
}

extern "C" const char* eps_measure_last_error() { return measure_error.c_str(); }
