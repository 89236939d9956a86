// index.hip -- device key -> slot index of one table (open addressing in HBM).
//
// The reference keeps a host hash map per table (CudaCacheBackend::Impl::Table
// ::rows, src/cuda/cache_backend.cu:193-198) and looks every key occurrence up
// in it on the host before a gather (:279-291).  Here the map lives in device
// memory beside the table, kept up to date by admissions and evictions, and a
// lookup resolves a whole batch of occurrences in one launch.
//
// Layout: `capacity` (a power of two) buckets of {u64 key, u64 slot}.  The slot
// word carries the bucket state: kEmpty, kGone (a removed entry, reused by
// later inserts), kClaimed (an insert in progress), or a slot.  Linear probing
// from a mixed hash of the key; a probe ends at the first empty bucket.
// Inserts and removals of one launch touch distinct keys (callers guarantee
// it); launches are stream ordered, so lookups never meet a partial insert.
// Nothing turns a kGone bucket back into kEmpty: under insert/remove churn
// they replace the empty buckets until a miss walks the whole cluster.  An
// owner that removes keys rebuilds the index (clear, then insert the live
// keys) after removals to a quarter of the buckets, which keeps at least a
// quarter of them empty at a load of at most one half.  HipCacheBackend does.
// (A removal that empties its bucket when the next one is empty was tried:
// under steady churn on a CPU model of this index it saved 5-10 % of a
// miss's probes and still lost every empty bucket, so it was left out.)
#include "common.hpp"

namespace eps_hip {
namespace {

constexpr uint64_t kEmpty = ~0ull;
constexpr uint64_t kGone = ~0ull - 1;
constexpr uint64_t kClaimed = ~0ull - 2;

struct Bucket {
  uint64_t key, slot;
};

__device__ __forceinline__ uint64_t Spread(uint64_t k) {  // a 64-bit finaliser (MurmurHash3 fmix64)
  k ^= k >> 33;
  k *= 0xff51afd7ed558ccdull;
  k ^= k >> 33;
  k *= 0xc4ceb9fe1a85ec53ull;
  return k ^ (k >> 33);
}

// Slot of `key`, or kEmpty when it is not in the index.
__device__ __forceinline__ uint64_t Find(const Bucket* b, uint64_t mask, uint64_t key) {
  uint64_t at = Spread(key) & mask;
  for (uint64_t probes = 0; probes <= mask; ++probes, at = (at + 1) & mask) {
    const uint64_t slot = b[at].slot;
    if (slot == kEmpty) return kEmpty;
    if (slot < kClaimed && b[at].key == key) return slot;
  }
  return kEmpty;
}

__global__ void InsertKernel(Bucket* b, uint64_t mask, const uint64_t* keys, const uint64_t* slots,
                             uint64_t count, uint32_t* status) {
  for (uint64_t i = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < count;
       i += uint64_t(blockDim.x) * gridDim.x) {
    const uint64_t key = keys[i], slot = slots[i];
    uint64_t at = Spread(key) & mask;
    bool placed = false;
    for (uint64_t probes = 0; probes <= mask && !placed; ++probes, at = (at + 1) & mask) {
      unsigned long long* word = reinterpret_cast<unsigned long long*>(&b[at].slot);
      unsigned long long seen = *word;
      if (seen != kEmpty && seen != kGone) continue;
      if (atomicCAS(word, seen, (unsigned long long)kClaimed) != seen) continue;
      b[at].key = key;
      __hip_atomic_store(word, (unsigned long long)slot, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      placed = true;
    }
    if (!placed && status) atomicOr(status, EPS_HIP_STATUS_BAD_INDEX);  // index full
  }
}

__global__ void RemoveKernel(Bucket* b, uint64_t mask, const uint64_t* keys, uint64_t count,
                             uint32_t* status) {
  for (uint64_t i = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < count;
       i += uint64_t(blockDim.x) * gridDim.x) {
    const uint64_t key = keys[i];
    uint64_t at = Spread(key) & mask;
    bool removed = false;
    for (uint64_t probes = 0; probes <= mask; ++probes, at = (at + 1) & mask) {
      const uint64_t slot = b[at].slot;
      if (slot == kEmpty) break;
      if (slot < kClaimed && b[at].key == key) {
        b[at].slot = kGone;
        removed = true;
        break;
      }
    }
    if (!removed && status) atomicOr(status, EPS_HIP_STATUS_BAD_INDEX);  // key was not indexed
  }
}

// Occurrence i -> slot.  With a caller's occurrence map: a hole stays a hole;
// otherwise the occurrence must name its unique row's key (unique_keys[u]),
// and that key must be in the index.  Without a map: the index decides (keys
// not in it become holes).  A mismatch reports BAD_INDEX and yields a hole.
__global__ void ResolveKernel(const Bucket* b, uint64_t mask, const uint64_t* keys, const uint64_t* occ2u,
                              const uint64_t* unique_keys, uint64_t unique_count, uint64_t n,
                              uint64_t* out, uint32_t* status) {
  bool bad = false;
  for (uint64_t i = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += uint64_t(blockDim.x) * gridDim.x) {
    const uint64_t key = keys[i];
    uint64_t result = kHole;
    if (occ2u) {
      const uint64_t u = occ2u[i];
      if (u != kHole) {
        if (u >= unique_count || unique_keys[u] != key) {
          bad = true;
        } else if (b) {
          result = Find(b, mask, key);
          if (result == kEmpty) { bad = true; result = kHole; }
        } else {
          result = u;  // rows carried with the request: the unique index is the source row
        }
      }
    } else if (b) {
      const uint64_t s = Find(b, mask, key);
      result = s == kEmpty ? kHole : s;
    }
    out[i] = result;
  }
  if (__ballot(bad) && (threadIdx.x & (kWave - 1)) == 0 && status) atomicOr(status, EPS_HIP_STATUS_BAD_INDEX);
}

unsigned Blocks(uint64_t n) {
  const uint64_t b = (n + kBlock - 1) / kBlock;
  return unsigned(b < 1 ? 1 : (b > 65536 ? 65536 : b));
}

int CheckIndex(const void* index, uint64_t capacity) {
  if (!index) return Fail(EPS_HIP_INVALID_ARGUMENT, "null key index");
  if (capacity < 2 || (capacity & (capacity - 1)))
    return Fail(EPS_HIP_INVALID_ARGUMENT, "key index capacity must be a power of two");
  if (reinterpret_cast<uintptr_t>(index) % 16) return Fail(EPS_HIP_INVALID_ARGUMENT, "key index must be 16-byte aligned");
  return EPS_HIP_OK;
}

}  // namespace
}  // namespace eps_hip

using namespace eps_hip;

extern "C" {

uint64_t eps_hip_index_bytes(uint64_t capacity) { return capacity * sizeof(Bucket); }

int eps_hip_index_clear(void* index, uint64_t capacity, void* stream) {
  EPS_HIP_TRY(CheckIndex(index, capacity));
  return LaunchFill(static_cast<uint32_t*>(index), 0xffffffffu, capacity * sizeof(Bucket) / 4, AsStream(stream));
}

int eps_hip_index_insert(void* index, uint64_t capacity, const uint64_t* keys, const uint64_t* slots,
                         uint64_t count, uint32_t* status, void* stream) {
  EPS_HIP_TRY(CheckIndex(index, capacity));
  if (!count) return EPS_HIP_OK;
  if (!keys || !slots) return Fail(EPS_HIP_INVALID_ARGUMENT, "null index insert buffers");
  hipLaunchKernelGGL(InsertKernel, dim3(Blocks(count)), dim3(kBlock), 0, AsStream(stream),
                     static_cast<Bucket*>(index), capacity - 1, keys, slots, count, status);
  EPS_HIP_LAUNCHED("index insert");
  return EPS_HIP_OK;
}

int eps_hip_index_remove(void* index, uint64_t capacity, const uint64_t* keys, uint64_t count,
                         uint32_t* status, void* stream) {
  EPS_HIP_TRY(CheckIndex(index, capacity));
  if (!count) return EPS_HIP_OK;
  if (!keys) return Fail(EPS_HIP_INVALID_ARGUMENT, "null index remove buffer");
  hipLaunchKernelGGL(RemoveKernel, dim3(Blocks(count)), dim3(kBlock), 0, AsStream(stream),
                     static_cast<Bucket*>(index), capacity - 1, keys, count, status);
  EPS_HIP_LAUNCHED("index remove");
  return EPS_HIP_OK;
}

int eps_hip_resolve(const void* index, uint64_t capacity, const uint64_t* keys, const uint64_t* occurrence_to_unique,
                    const uint64_t* unique_keys, uint64_t unique_count, uint64_t n, uint64_t* slots,
                    uint32_t* status, void* stream) {
  if (index) EPS_HIP_TRY(CheckIndex(index, capacity));
  if (!n) return EPS_HIP_OK;
  if (!keys || !slots || (occurrence_to_unique && unique_count && !unique_keys) || (!index && !occurrence_to_unique))
    return Fail(EPS_HIP_INVALID_ARGUMENT, "invalid occurrence resolution arguments");
  hipLaunchKernelGGL(ResolveKernel, dim3(Blocks(n)), dim3(kBlock), 0, AsStream(stream),
                     static_cast<const Bucket*>(index), index ? capacity - 1 : 0, keys, occurrence_to_unique,
                     unique_keys, unique_count, n, slots, status);
  EPS_HIP_LAUNCHED("resolve occurrences");
  return EPS_HIP_OK;
}

}  // extern "C"
