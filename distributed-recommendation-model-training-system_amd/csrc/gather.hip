// gather.hip -- pooled gather (pull), row-state movement and initialisation.
//
// Pull = one launch for up to 32 features.  A block owns a tile of output rows
// (bags, or positions for sequence pooling) of one feature.  It stages the
// tile's bag offsets and row slots in LDS (one coalesced pass, unique->slot
// remap and range checks done once per occurrence), then sub-wavefront groups
// of G = dim/4 lanes (rounded up to a power of two, 4..64) each own one output
// row: lane l holds columns [4l, 4l+4) and adds the bag's rows with 128-bit
// loads, strictly in occurrence order from +0.0f, as the reference does
// (GatherKernel, src/cuda/cache_backend.cu:81-94; PrepareFeature,
// src/access/batch_access.cpp:41-50).  The mean divide of the client
// (src/client/distributed_client.cpp:227-232; NormalizeMean,
// src/cuda/cache_backend.cu:134-139) is fused into the store.
#include "common.hpp"

#include <algorithm>
#include <cfloat>
#include <mutex>

namespace eps_hip {

static thread_local std::string g_error;
void SetError(const std::string& message) { g_error = message; }
int Fail(int code, const std::string& message) { g_error = message; return code; }
int Check(hipError_t e, const char* what) {
  if (e == hipSuccess) return EPS_HIP_OK;
  g_error = std::string(what) + ": " + hipGetErrorString(e);
  return e == hipErrorOutOfMemory ? EPS_HIP_CAPACITY_EXCEEDED : EPS_HIP_RUN_FAILED;
}

namespace {

constexpr uint32_t kIdCap = 1024;     // occurrences staged in LDS per tile (LDS sets the occupancy)
constexpr uint32_t kGatherBatch = 8;  // source rows in flight per lane group
constexpr uint32_t kGenericLog2 = 0xff;
constexpr int kBufferWord3 = 0x00020000;         // raw buffer resource, dword data (gfx9 family)
constexpr uint32_t kBufferOutside = 0xFFFFFFF0u;  // an offset past every buffer range
typedef int EpsI4 __attribute__((ext_vector_type(4)));

struct GatherDesc {
  const float* source;
  const uint64_t* indices;
  const uint64_t* remap;
  const uint64_t* offsets;
  const uint64_t* lengths;
  const float* weights;
  float* output;
  uint64_t stride, rows, source_rows, remap_count;
  uint32_t dim, pooling, block_begin, log2g, rows_per_block;
  // Bytes of the source when they fit a 32-bit buffer range (0: they do not):
  // the row loads then go through a buffer resource, and the slots of a batch
  // past the bag's end (or holes) take an offset outside the range, which
  // returns zeros without a memory request.
  uint32_t buffer_bytes;
};
struct GatherArgs {
  GatherDesc part[EPS_HIP_MAX_GATHER_PARTS];
  uint32_t count;
  uint32_t* status;
};
static_assert(sizeof(GatherArgs) <= 4096, "gather arguments fit the kernel-argument segment");

// Slot of occurrence `i` (or kHole); range failures are reported and skipped.
__device__ __forceinline__ uint64_t ResolveSlot(const GatherDesc& d, uint64_t i, bool& bad) {
  uint64_t idx = d.indices[i];
  if (idx == kHole) return kHole;
  if (d.remap) {
    if (idx >= d.remap_count) { bad = true; return kHole; }
    idx = d.remap[idx];
  }
  if (idx >= d.source_rows) { bad = true; return kHole; }
  return idx;
}

__global__ void __launch_bounds__(kBlock) GatherKernel(GatherArgs args) {
  const GatherDesc d = args.part[PartOf(args.part, args.count)];

  __shared__ uint64_t s_off[129];
  __shared__ uint64_t s_slot[kIdCap];
  __shared__ float s_weight[kIdCap];
  __shared__ uint32_t s_bad;

  const bool seq = d.pooling == EPS_HIP_POOL_SEQUENCE;
  const bool weighted = d.pooling == EPS_HIP_POOL_WEIGHTED_SUM;
  const uint64_t row0 = uint64_t(blockIdx.x - d.block_begin) * d.rows_per_block;
  if (row0 >= d.rows) return;
  const uint64_t row_end = min(row0 + d.rows_per_block, d.rows);
  const uint32_t nrows = uint32_t(row_end - row0);
  if (threadIdx.x == 0) s_bad = 0;
  if (!seq)
    for (uint32_t r = threadIdx.x; r <= nrows; r += kBlock) s_off[r] = d.offsets[row0 + r];
  __syncthreads();
  const uint64_t occ_begin = seq ? row0 : s_off[0];
  // A part without indices has no occurrences (every bag empty): nothing is
  // read, and offsets that claim occurrences are reported as bad indices.
  const bool none = d.indices == nullptr;
  if (none && !seq && s_off[nrows] != s_off[0] && threadIdx.x == 0) s_bad = 1;
  const uint64_t occ_end = none ? occ_begin : (seq ? row_end : s_off[nrows]);
  const bool staged = occ_end - occ_begin <= kIdCap;
  bool bad = false;
  if (staged) {
    for (uint64_t i = occ_begin + threadIdx.x; i < occ_end; i += kBlock) {
      s_slot[i - occ_begin] = ResolveSlot(d, i, bad);
      if (weighted) s_weight[i - occ_begin] = d.weights[i];
    }
  }
  __syncthreads();

  if (d.log2g != kGenericLog2) {
    const uint32_t G = 1u << d.log2g;
    const uint32_t lig = threadIdx.x & (G - 1);
    const uint32_t ngroups = kBlock >> d.log2g;
    const uint32_t c = lig * 4;
    const bool active = c < d.dim;
    for (uint32_t r = threadIdx.x >> d.log2g; r < nrows; r += ngroups) {
      const uint64_t beg = seq ? row0 + r : s_off[r];
      const uint64_t end = none ? beg : (seq ? row0 + r + 1 : s_off[r + 1]);
      float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
      if (staged && d.source_rows) {
        // Staged slots: every load of a batch is issued before any is added,
        // with no branch around a load (a hole or a position past the bag
        // reads row 0, column 0 and is dropped; row 0 exists).
        const uint32_t cl = active ? c : 0;
        const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<float*>(d.source), (short)0, int(d.buffer_bytes), kBufferWord3);
        for (uint64_t pos = beg; pos < end; pos += kGatherBatch) {
          float4 v[kGatherBatch];
          float a[kGatherBatch];
          bool ok[kGatherBatch];
#pragma unroll
          for (uint32_t u = 0; u < kGatherBatch; ++u) {
            const uint64_t i = pos + u;
            const uint32_t at = uint32_t(min(i, end - 1) - occ_begin);
            const uint64_t slot = s_slot[at];
            ok[u] = i < end && slot != kHole;
            a[u] = weighted ? s_weight[at] : 1.f;
            if (d.buffer_bytes) {
              const uint32_t boff = ok[u] && active ? uint32_t((slot * d.stride + c) * 4) : kBufferOutside;
              const EpsI4 q = __builtin_amdgcn_raw_buffer_load_b128(rsrc, boff, 0, 0);
              v[u] = make_float4(__int_as_float(q[0]), __int_as_float(q[1]), __int_as_float(q[2]),
                                 __int_as_float(q[3]));
            } else {
              v[u] = Load4(d.source + (ok[u] ? slot : 0) * d.stride + cl);
            }
          }
#pragma unroll
          for (uint32_t u = 0; u < kGatherBatch; ++u) {
            if (!ok[u]) continue;
            if (weighted) {
              acc.x += v[u].x * a[u]; acc.y += v[u].y * a[u];
              acc.z += v[u].z * a[u]; acc.w += v[u].w * a[u];
            } else {
              acc.x += v[u].x; acc.y += v[u].y; acc.z += v[u].z; acc.w += v[u].w;
            }
          }
        }
      } else {
        for (uint64_t pos = beg; pos < end; pos += 4) {
          float4 v[4];
          float a[4];
          bool ok[4];
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            const uint64_t i = pos + u;
            uint64_t slot = kHole;
            a[u] = 1.f;
            if (i < end) {
              if (staged) {
                slot = s_slot[i - occ_begin];
                if (weighted) a[u] = s_weight[i - occ_begin];
              } else {
                slot = ResolveSlot(d, i, bad);
                if (weighted) a[u] = d.weights[i];
              }
            }
            ok[u] = slot != kHole;
            v[u] = (ok[u] && active) ? Load4(d.source + slot * d.stride + c)
                                     : make_float4(0.f, 0.f, 0.f, 0.f);
          }
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            if (!ok[u]) continue;
            if (weighted) {
              acc.x += v[u].x * a[u]; acc.y += v[u].y * a[u];
              acc.z += v[u].z * a[u]; acc.w += v[u].w * a[u];
            } else {
              acc.x += v[u].x; acc.y += v[u].y; acc.z += v[u].z; acc.w += v[u].w;
            }
          }
        }
      }
      if (d.pooling == EPS_HIP_POOL_MEAN && d.lengths) {
        const uint64_t len = d.lengths[row0 + r];
        if (len) {
          const float f = (float)len;
          acc.x = acc.x / f; acc.y = acc.y / f; acc.z = acc.z / f; acc.w = acc.w / f;
        }
      }
      if (active) Store4(d.output + (row0 + r) * d.dim + c, acc);
    }
  } else {
    // Generic shapes (dim % 4 != 0 or dim > 256): one wavefront per row,
    // scalar columns, same per-column operation order.
    const uint32_t lane = threadIdx.x & (kWave - 1);
    for (uint32_t r = threadIdx.x / kWave; r < nrows; r += kBlock / kWave) {
      const uint64_t beg = seq ? row0 + r : s_off[r];
      const uint64_t end = none ? beg : (seq ? row0 + r + 1 : s_off[r + 1]);
      float div = 0.f;
      if (d.pooling == EPS_HIP_POOL_MEAN && d.lengths) div = (float)d.lengths[row0 + r];
      for (uint32_t c = lane; c < d.dim; c += kWave) {
        float acc = 0.f;
        for (uint64_t i = beg; i < end; ++i) {
          const uint64_t slot = staged ? s_slot[i - occ_begin] : ResolveSlot(d, i, bad);
          if (slot == kHole) continue;
          const float x = d.source[slot * d.stride + c];
          if (weighted) acc += x * (staged ? s_weight[i - occ_begin] : d.weights[i]);
          else acc += x;
        }
        if (div != 0.f) acc = acc / div;
        d.output[(row0 + r) * d.dim + c] = acc;
      }
    }
  }
  if (bad) s_bad = 1;
  __syncthreads();
  if (threadIdx.x == 0 && s_bad && args.status) atomicOr(args.status, EPS_HIP_STATUS_BAD_INDEX);
}

__global__ void AddContributionKernel(float* output, const float* source, const uint64_t* positions,
                                      uint64_t values, uint32_t dim) {
  for (uint64_t i = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < values;
       i += uint64_t(blockDim.x) * gridDim.x) {
    const uint64_t target = positions ? positions[i / dim] * dim + i % dim : i;
    output[target] += source[i];
  }
}

// NormalizeMean (src/cuda/cache_backend.cu:134-139): output[r, d] /= len[r]
// for len[r] != 0, an IEEE float divide by the length converted to float.
__global__ void NormalizeMeanKernel(float* output, const uint64_t* lengths, uint64_t rows,
                                    uint32_t dim) {
  const uint64_t values = rows * dim;
  for (uint64_t i = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < values;
       i += uint64_t(blockDim.x) * gridDim.x) {
    const uint64_t len = lengths[i / dim];
    if (len) output[i] = output[i] / (float)len;
  }
}

// target[i] = value for i < count, except i == keep (kept as it is).
__global__ void FillKernel(uint32_t* target, uint32_t value, uint64_t count, uint64_t keep) {
  for (uint64_t i = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < count;
       i += uint64_t(blockDim.x) * gridDim.x)
    if (i != keep) target[i] = value;
}

__device__ __forceinline__ uint64_t Mix(uint64_t x) {
  x += 0x9e3779b97f4a7c15ULL;
  x = (x ^ (x >> 30)) * 0xbf58476d1ce4e5b9ULL;
  x = (x ^ (x >> 27)) * 0x94d049bb133111ebULL;
  return x ^ (x >> 31);
}

__device__ __forceinline__ void BoundMax(Bounds* bounds, uint32_t w, uint32_t m, uint32_t v) {
  w = WaveMax(w); m = WaveMax(m); v = WaveMax(v);
  if ((threadIdx.x & (kWave - 1)) == 0 && bounds) {
    uint32_t* slot = bounds->v[(blockIdx.x * (kBlock / kWave) + threadIdx.x / kWave) % kBoundSlots];
    if (w) atomicMax(slot + 0, w);
    if (m) atomicMax(slot + 1, m);
    if (v) atomicMax(slot + 2, v);
  }
}

// ShardStore::Ensure's initializer (src/store/shard_store.cpp:104-112) for
// key = key_base + slot * key_stride; salt = Mix(seed) ^ Mix(table id).
__global__ void InitRowsKernel(float* state, uint32_t dim, uint64_t first, uint64_t count,
                               uint64_t key_base, uint64_t key_stride, uint64_t salt,
                               double lo, double hi, int32_t bounded, float wmin, float wmax,
                               Bounds* bounds) {
  uint32_t wmax_bits = 0;
  const uint64_t total = count * dim;
  for (uint64_t e = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x; e < total;
       e += uint64_t(blockDim.x) * gridDim.x) {
    const uint64_t slot = first + e / dim;
    const uint32_t col = uint32_t(e % dim);
    const uint64_t key = key_base + slot * key_stride;
    const uint64_t bits = Mix(key ^ salt ^ Mix(uint64_t(col)));
    const double u = double(bits >> 11) * 0x1.0p-53;
    float w = float((1 - u) * lo + u * hi);
    if (bounded) w = Clamp(w, wmin, wmax);
    float* row = state + slot * uint64_t(dim) * 3;
    row[col] = w;
    row[dim + col] = 0.f;
    row[2 * dim + col] = 0.f;
    wmax_bits = max(wmax_bits, AbsBits(w));
  }
  BoundMax(bounds, wmax_bits, 0, 0);
}

// ScatterState (src/cuda/cache_backend.cu:69-74): packed [w|m|v] rows -> slots.
__global__ void ScatterRowsKernel(float* state, uint32_t dim, const uint64_t* slots,
                                  const float* packed, uint64_t count, Bounds* bounds) {
  uint32_t bw = 0, bm = 0, bv = 0;
  const uint64_t width = uint64_t(dim) * 3;
  if ((dim & 3) == 0) {
    const uint64_t w4 = width / 4, total = count * w4;
    for (uint64_t e = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x; e < total;
         e += uint64_t(blockDim.x) * gridDim.x) {
      const uint64_t row = e / w4, col = (e % w4) * 4;
      const float4 x = Load4(packed + row * width + col);
      Store4(state + slots[row] * width + col, x);
      const uint32_t a = max(max(AbsBits(x.x), AbsBits(x.y)), max(AbsBits(x.z), AbsBits(x.w)));
      if (col < dim) bw = max(bw, a); else if (col < 2 * dim) bm = max(bm, a); else bv = max(bv, a);
    }
  } else {
    const uint64_t total = count * width;
    for (uint64_t e = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x; e < total;
         e += uint64_t(blockDim.x) * gridDim.x) {
      const uint64_t row = e / width, col = e % width;
      const float x = packed[e];
      state[slots[row] * width + col] = x;
      if (col < dim) bw = max(bw, AbsBits(x)); else if (col < 2 * dim) bm = max(bm, AbsBits(x));
      else bv = max(bv, AbsBits(x));
    }
  }
  BoundMax(bounds, bw, bm, bv);
}

// ReadStateKernel (src/cuda/cache_backend.cu:75-80): slots -> packed rows.
__global__ void GatherRowsKernel(const float* state, uint32_t dim, const uint64_t* slots,
                                 float* packed, uint64_t count) {
  const uint64_t width = uint64_t(dim) * 3;
  if ((dim & 3) == 0) {
    const uint64_t w4 = width / 4, total = count * w4;
    for (uint64_t e = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x; e < total;
         e += uint64_t(blockDim.x) * gridDim.x) {
      const uint64_t row = e / w4, col = (e % w4) * 4;
      Store4(packed + row * width + col, Load4(state + slots[row] * width + col));
    }
  } else {
    const uint64_t total = count * width;
    for (uint64_t e = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x; e < total;
         e += uint64_t(blockDim.x) * gridDim.x)
      packed[e] = state[slots[e / width] * width + e % width];
  }
}

// Row moves of several tables in one launch (admissions: packed -> slots,
// like ScatterRowsKernel; write-backs: slots -> packed, like
// GatherRowsKernel).  A part's 16-byte pieces (scalar floats when dim % 4)
// form chunks of kBlock * kMovePerThread; the launch's blocks take the chunks
// of all parts in turn (chunk c, c + gridDim.x, ...).  When one side is host
// memory the grid is small: each block's loads wait microseconds on the host
// link, and a few blocks keep enough bytes in flight for it without holding
// wave slots the step's own kernels need.
constexpr uint32_t kMovePerThread = 4;
constexpr uint32_t kHostLinkGrid = 16;  // blocks of a move that crosses the host link (best of 8-64 on
                                         // config 5: fewer slow the moves, more slow the step)
struct MoveDesc {
  float* state;
  float* packed;
  const uint64_t* slots;
  uint64_t count;
  uint32_t dim, block_begin;  // block_begin: the part's first chunk
};
struct MoveArgs {
  MoveDesc part[EPS_HIP_MAX_TABLES];
  uint32_t count, chunks;
  uint32_t write_back;
  Bounds* bounds;
};

__global__ void __launch_bounds__(kBlock) MoveRowsKernel(MoveArgs a) {
  uint32_t bw = 0, bm = 0, bv = 0;
  for (uint32_t chunk = blockIdx.x; chunk < a.chunks; chunk += gridDim.x) {
    const MoveDesc d = a.part[PartOf(a.part, a.count, chunk)];
    const uint64_t width = uint64_t(d.dim) * 3;
    const bool vec = (d.dim & 3) == 0;
    const uint64_t per_row = vec ? width / 4 : width;
    const uint64_t items = d.count * per_row;
    const uint64_t first = uint64_t(chunk - d.block_begin) * kBlock * kMovePerThread;
    // Every load of the thread is issued before any store: one side may be
    // host memory, microseconds away over the host link.
    const float* src[kMovePerThread];
    float* dst[kMovePerThread];
    uint64_t col[kMovePerThread];
    bool ok[kMovePerThread];
#pragma unroll
    for (uint32_t k = 0; k < kMovePerThread; ++k) {
      const uint64_t e = first + uint64_t(k) * kBlock + threadIdx.x;
      ok[k] = e < items;
      const uint64_t row = ok[k] ? e / per_row : 0, piece = ok[k] ? e % per_row : 0;
      col[k] = vec ? piece * 4 : piece;
      float* slot_row = d.state + (ok[k] ? d.slots[row] : 0) * width + col[k];
      float* packed = d.packed + row * width + col[k];
      src[k] = a.write_back ? slot_row : packed;
      dst[k] = a.write_back ? packed : slot_row;
    }
    if (vec) {
      float4 x[kMovePerThread];
#pragma unroll
      for (uint32_t k = 0; k < kMovePerThread; ++k) x[k] = ok[k] ? Load4(src[k]) : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
      for (uint32_t k = 0; k < kMovePerThread; ++k) {
        if (!ok[k]) continue;
        Store4(dst[k], x[k]);
        const uint32_t m = max(max(AbsBits(x[k].x), AbsBits(x[k].y)), max(AbsBits(x[k].z), AbsBits(x[k].w)));
        if (col[k] < d.dim) bw = max(bw, m); else if (col[k] < 2 * d.dim) bm = max(bm, m); else bv = max(bv, m);
      }
    } else {
      float x[kMovePerThread];
#pragma unroll
      for (uint32_t k = 0; k < kMovePerThread; ++k) x[k] = ok[k] ? LoadF(src[k]) : 0.f;
#pragma unroll
      for (uint32_t k = 0; k < kMovePerThread; ++k) {
        if (!ok[k]) continue;
        StoreF(dst[k], x[k]);
        if (col[k] < d.dim) bw = max(bw, AbsBits(x[k])); else if (col[k] < 2 * d.dim) bm = max(bm, AbsBits(x[k]));
        else bv = max(bv, AbsBits(x[k]));
      }
    }
  }
  if (!a.write_back) BoundMax(a.bounds, bw, bm, bv);
}

unsigned GridFor(uint64_t n, unsigned cap = 65536) {
  const uint64_t blocks = (n + kBlock - 1) / kBlock;
  return unsigned(blocks < 1 ? 1 : (blocks > cap ? cap : blocks));
}

uint64_t HostMix(uint64_t x) {
  x += 0x9e3779b97f4a7c15ULL;
  x = (x ^ (x >> 30)) * 0xbf58476d1ce4e5b9ULL;
  x = (x ^ (x >> 27)) * 0x94d049bb133111ebULL;
  return x ^ (x >> 31);
}

// Device-visible address of a row buffer: device memory as is, pinned host
// memory through its mapped device pointer; pageable host memory is refused
// (a kernel must never dereference an unmapped host address).
int DeviceAddress(const void* p, const void** out, bool* host = nullptr) {
  hipPointerAttribute_t attr;
  if (hipPointerGetAttributes(&attr, p) != hipSuccess) {
    (void)hipGetLastError();
    return Fail(EPS_HIP_INVALID_ARGUMENT, "row buffer must be device memory or pinned host memory");
  }
  if (host) *host = attr.type == hipMemoryTypeHost;
  if (attr.type == hipMemoryTypeHost) {
    if (!attr.devicePointer) return Fail(EPS_HIP_INVALID_ARGUMENT, "pinned host buffer is not mapped");
    *out = attr.devicePointer;
  } else {
    *out = p;
  }
  return EPS_HIP_OK;
}

int CheckTable(const eps_hip_table* t) {
  if (!t || !t->state) return Fail(EPS_HIP_INVALID_ARGUMENT, "null table");
  if (t->dim == 0 || t->dim > 65536) return Fail(EPS_HIP_INVALID_ARGUMENT, "invalid dimension");
  if (reinterpret_cast<uintptr_t>(t->state) % 16)
    return Fail(EPS_HIP_INVALID_ARGUMENT, "table state must be 16-byte aligned");
  return EPS_HIP_OK;
}

}  // namespace

int LaunchFill(uint32_t* target, uint32_t value, uint64_t count, hipStream_t stream, uint64_t keep) {
  if (!count) return EPS_HIP_OK;
  hipLaunchKernelGGL(FillKernel, dim3(GridFor(count, 4096)), dim3(kBlock), 0, stream, target,
                     value, count, keep);
  EPS_HIP_LAUNCHED("fill");
  return EPS_HIP_OK;
}

}  // namespace eps_hip

using namespace eps_hip;

extern "C" {

int eps_hip_abi_version(void) { return EPS_HIP_ABI_VERSION; }
const char* eps_hip_last_error(void) { return g_error.c_str(); }

int eps_hip_device_check(int device) {
  EPS_HIP_TRY(Check(hipSetDevice(device), "hipSetDevice"));
  hipDeviceProp_t prop;
  EPS_HIP_TRY(Check(hipGetDeviceProperties(&prop, device), "hipGetDeviceProperties"));
  if (std::string(prop.gcnArchName).rfind("gfx950", 0) != 0)
    return Fail(EPS_HIP_UNAVAILABLE, std::string("device is ") + prop.gcnArchName + ", not gfx950");
  return EPS_HIP_OK;
}

uint64_t eps_hip_bounds_bytes(void) { return sizeof(Bounds); }

int eps_hip_bounds_reset(void* bounds, void* stream) {
  if (!bounds) return Fail(EPS_HIP_INVALID_ARGUMENT, "null bounds");
  return LaunchFill(static_cast<uint32_t*>(bounds), 0, sizeof(Bounds) / 4, AsStream(stream));
}

int eps_hip_fill_u32(uint32_t* target, uint32_t value, uint64_t count, void* stream) {
  if (!target && count) return Fail(EPS_HIP_INVALID_ARGUMENT, "null target");
  return LaunchFill(target, value, count, AsStream(stream));
}

int eps_hip_init_rows(const eps_hip_table* t, uint64_t first, uint64_t count, uint64_t key_base,
                      uint64_t key_stride, uint64_t seed, float init_min, float init_max,
                      int32_t bounded, float weight_min, float weight_max, void* bounds,
                      void* stream) {
  EPS_HIP_TRY(CheckTable(t));
  if (first > t->rows || count > t->rows - first)
    return Fail(EPS_HIP_INVALID_ARGUMENT, "initialised slots exceed table rows");
  if (!count) return EPS_HIP_OK;
  const uint64_t salt = HostMix(seed) ^ HostMix(uint64_t(t->id));
  hipLaunchKernelGGL(InitRowsKernel, dim3(GridFor(count * t->dim)), dim3(kBlock), 0,
                     AsStream(stream), t->state, t->dim, first, count, key_base, key_stride, salt,
                     double(init_min), double(init_max), bounded, weight_min, weight_max,
                     static_cast<Bounds*>(bounds));
  EPS_HIP_LAUNCHED("init rows");
  return EPS_HIP_OK;
}

int eps_hip_scatter_rows(const eps_hip_table* t, const uint64_t* slots, const float* packed,
                         uint64_t count, void* bounds, void* stream) {
  EPS_HIP_TRY(CheckTable(t));
  if (!count) return EPS_HIP_OK;
  if (!slots || !packed) return Fail(EPS_HIP_INVALID_ARGUMENT, "null scatter buffers");
  const void* source = nullptr;
  EPS_HIP_TRY(DeviceAddress(packed, &source));
  packed = static_cast<const float*>(source);
  const uint64_t work = (t->dim % 4 == 0) ? count * t->dim * 3 / 4 : count * t->dim * 3;
  hipLaunchKernelGGL(ScatterRowsKernel, dim3(GridFor(work)), dim3(kBlock), 0, AsStream(stream),
                     t->state, t->dim, slots, packed, count, static_cast<Bounds*>(bounds));
  EPS_HIP_LAUNCHED("scatter rows");
  return EPS_HIP_OK;
}

int eps_hip_gather_rows(const eps_hip_table* t, const uint64_t* slots, float* packed,
                        uint64_t count, void* stream) {
  EPS_HIP_TRY(CheckTable(t));
  if (!count) return EPS_HIP_OK;
  if (!slots || !packed) return Fail(EPS_HIP_INVALID_ARGUMENT, "null gather buffers");
  const void* target = nullptr;
  EPS_HIP_TRY(DeviceAddress(packed, &target));
  packed = static_cast<float*>(const_cast<void*>(target));
  const uint64_t work = (t->dim % 4 == 0) ? count * t->dim * 3 / 4 : count * t->dim * 3;
  hipLaunchKernelGGL(GatherRowsKernel, dim3(GridFor(work)), dim3(kBlock), 0, AsStream(stream),
                     t->state, t->dim, slots, packed, count);
  EPS_HIP_LAUNCHED("gather rows");
  return EPS_HIP_OK;
}

int eps_hip_move_rows(const eps_hip_row_batch* batches, uint32_t count, int32_t write_back, void* bounds,
                      void* stream) {
  if (count > EPS_HIP_MAX_TABLES) return Fail(EPS_HIP_INVALID_ARGUMENT, "too many row batches");
  if (count && !batches) return Fail(EPS_HIP_INVALID_ARGUMENT, "null row batches");
  MoveArgs args{};
  args.write_back = write_back ? 1u : 0u;
  args.bounds = static_cast<Bounds*>(bounds);
  uint64_t blocks = 0;
  bool host_link = false;
  for (uint32_t i = 0; i < count; ++i) {
    const eps_hip_row_batch& b = batches[i];
    if (!b.count) continue;
    if (!b.state || !b.slots || !b.packed || b.dim == 0 || b.dim > 65536)
      return Fail(EPS_HIP_INVALID_ARGUMENT, "invalid row batch");
    if (reinterpret_cast<uintptr_t>(b.state) % 16) return Fail(EPS_HIP_INVALID_ARGUMENT, "table state must be 16-byte aligned");
    const void* packed = nullptr;
    bool host = false;
    EPS_HIP_TRY(DeviceAddress(b.packed, &packed, &host));
    host_link = host_link || host;
    if ((b.dim & 3) == 0 && reinterpret_cast<uintptr_t>(packed) % 16)
      return Fail(EPS_HIP_INVALID_ARGUMENT, "packed rows must be 16-byte aligned");
    MoveDesc& d = args.part[args.count++];
    d.state = b.state;
    d.packed = static_cast<float*>(const_cast<void*>(packed));
    d.slots = b.slots;
    d.count = b.count;
    d.dim = b.dim;
    d.block_begin = uint32_t(blocks);
    const uint64_t per_row = (b.dim & 3) == 0 ? uint64_t(b.dim) * 3 / 4 : uint64_t(b.dim) * 3;
    blocks += (b.count * per_row + kBlock * kMovePerThread - 1) / (kBlock * kMovePerThread);
    if (blocks >= (1ull << 31)) return Fail(EPS_HIP_CAPACITY_EXCEEDED, "row move grid too large");
  }
  if (!blocks) return EPS_HIP_OK;
  args.chunks = uint32_t(blocks);
  const uint64_t grid = std::min<uint64_t>(blocks, host_link ? kHostLinkGrid : 65536);
  hipLaunchKernelGGL(MoveRowsKernel, dim3(unsigned(grid)), dim3(kBlock), 0, AsStream(stream), args);
  EPS_HIP_LAUNCHED("move rows");
  return EPS_HIP_OK;
}

int eps_hip_gather(const eps_hip_gather_part* parts, uint32_t count, uint32_t* status,
                   void* stream) {
  if (count > EPS_HIP_MAX_GATHER_PARTS) return Fail(EPS_HIP_INVALID_ARGUMENT, "too many gather parts");
  GatherArgs args{};
  args.status = status;
  uint32_t blocks = 0, used = 0;
  for (uint32_t p = 0; p < count; ++p) {
    const auto& in = parts[p];
    if (in.dim == 0 || in.pooling > EPS_HIP_POOL_WEIGHTED_SUM)
      return Fail(EPS_HIP_INVALID_ARGUMENT, "invalid gather part");
    if (in.rows == 0) continue;
    // indices (and weights) may be NULL only for a pooled part whose bags are
    // all empty; offsets that claim occurrences then raise the bad-index bit.
    if (!in.source || !in.output || (in.pooling == EPS_HIP_POOL_SEQUENCE && !in.indices) ||
        (in.pooling != EPS_HIP_POOL_SEQUENCE && !in.offsets) ||
        (in.pooling == EPS_HIP_POOL_WEIGHTED_SUM && in.indices && !in.weights))
      return Fail(EPS_HIP_INVALID_ARGUMENT, "null gather buffer");
    GatherDesc& d = args.part[used++];
    d.source = in.source; d.indices = in.indices; d.remap = in.remap; d.offsets = in.offsets;
    d.lengths = in.valid_lengths; d.weights = in.weights; d.output = in.output;
    d.stride = in.stride; d.rows = in.rows; d.source_rows = in.source_rows;
    d.remap_count = in.remap_count; d.dim = in.dim; d.pooling = in.pooling;
    const uint64_t source_bytes = in.source_rows * in.stride * 4;
    d.buffer_bytes = source_bytes && source_bytes < kBufferOutside && in.source_rows < (1ull << 32)
                         ? uint32_t(source_bytes) : 0u;
    const bool vec = in.dim % 4 == 0 && in.dim <= 256 && in.stride % 4 == 0 &&
                     reinterpret_cast<uintptr_t>(in.source) % 16 == 0 &&
                     reinterpret_cast<uintptr_t>(in.output) % 16 == 0;
    if (vec) {
      uint32_t log2g = 2;
      while ((1u << log2g) < in.dim / 4) ++log2g;
      d.log2g = log2g;
      d.rows_per_block = kBlock >> log2g;  // one bag per lane group
    } else {
      d.log2g = kGenericLog2;
      d.rows_per_block = 8;
    }
    d.block_begin = blocks;
    const uint64_t b = (in.rows + d.rows_per_block - 1) / d.rows_per_block;
    if (b > (1ull << 31) - blocks) return Fail(EPS_HIP_CAPACITY_EXCEEDED, "gather grid too large");
    blocks += uint32_t(b);
  }
  args.count = used;
  if (!blocks) return EPS_HIP_OK;
  hipLaunchKernelGGL(GatherKernel, dim3(blocks), dim3(kBlock), 0, AsStream(stream), args);
  EPS_HIP_LAUNCHED("gather");
  return EPS_HIP_OK;
}

int eps_hip_normalize_mean(float* output, const uint64_t* lengths, uint64_t rows, uint32_t dim,
                           void* stream) {
  if (!rows) return EPS_HIP_OK;
  if (!output || !lengths || !dim) return Fail(EPS_HIP_INVALID_ARGUMENT, "invalid mean normalisation");
  hipLaunchKernelGGL(NormalizeMeanKernel, dim3(GridFor(rows * dim)), dim3(kBlock), 0,
                     AsStream(stream), output, lengths, rows, dim);
  EPS_HIP_LAUNCHED("normalize mean");
  return EPS_HIP_OK;
}

int eps_hip_add_contribution(float* output, const float* source, const uint64_t* positions,
                             uint64_t values, uint32_t dim, void* stream) {
  if (!values) return EPS_HIP_OK;
  if (!output || !source || !dim) return Fail(EPS_HIP_INVALID_ARGUMENT, "invalid contribution");
  hipLaunchKernelGGL(AddContributionKernel, dim3(GridFor(values)), dim3(kBlock), 0,
                     AsStream(stream), output, source, positions, values, dim);
  EPS_HIP_LAUNCHED("add contribution");
  return EPS_HIP_OK;
}

}  // extern "C"
