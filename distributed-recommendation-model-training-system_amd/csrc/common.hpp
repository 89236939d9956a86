// common.hpp -- shared definitions of the gfx950 kernel library (libeps_hip.so).
#pragma once
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <cstdio>
#include <string>

#include "eps_hip.h"
#include "guard.hpp"

namespace eps_hip {

constexpr uint32_t kBlock = 256;          // 4 wavefronts of 64
constexpr uint32_t kWave = 64;
constexpr uint64_t kHole = ~0ull;         // "row not on this device" (UINT64_MAX)
constexpr uint32_t kBoundSlots = 64;      // spread of the bound atomics
constexpr uint32_t kSortTile = 4096;      // keys per radix-sort tile (256 x 16)
constexpr uint32_t kSortItems = 16;
constexpr uint32_t kGroupTiles = 16;     // radix tiles per look-back group
constexpr uint32_t kMaxPasses = 4;
constexpr uint32_t kRadixBits = 9;        // largest radix digit
constexpr uint32_t kDigits = 1u << kRadixBits;
constexpr uint32_t kDigitsPerThread = kDigits / kBlock;  // the sort kernels assume two
static_assert(kDigitsPerThread == 2, "radix digits per thread");
constexpr uint32_t kKeygenItems = 8;      // occurrences per keygen thread
constexpr uint32_t kClasses = 6;          // 5 vector widths + generic
constexpr uint32_t kRefRowBits = 27;      // gradient row bits in a reference word
static_assert(kRefRowBits == kGuardRefRowBits, "one reference word layout");
constexpr uint32_t kLongRefs = 128;       // rows with more references take the sliced path

constexpr uint32_t kSrcSlots = 64;        // spread of the gradient/scale maximum atomics
constexpr uint32_t kHistCopies = 16;      // spread of the keygen histogram atomics
constexpr uint32_t kXcds = 8;             // XCDs of an MI355X
constexpr uint32_t kHotBuckets = 8;       // hot-row lists per XCD, by length (longest first)

// Control block at offset 0 of a push or update workspace (1 KiB).  Values
// that many blocks update are kept in several copies (slots) written round
// robin and combined by their reader: atomics that all blocks aim at one
// address serialise in the memory-side atomic unit.
struct Control {
  uint32_t status;          // result of the last push/update (0 = applied)
  uint32_t prep_status;     // prepare-time findings (bad slots, bad scales)
  uint32_t src_slots[kSrcSlots];    // max |gradient| as float bits, per slot
  uint32_t scale_slots[kSrcSlots];  // max |scale| above 1.0 as float bits, per slot
  uint32_t valid_count;     // prepared occurrences that are on this device
  uint32_t mode;            // guard decision of the last push
  uint32_t reserved;
  uint32_t unique_count;
  uint32_t tile_counter[kMaxPasses];
  uint32_t class_start[8];  // first sorted position of each dimension class (+ end)
  uint32_t long_count[kXcds * kHotBuckets];  // entries of each hot-row list
  // Bounds-domain maxima W, M, V as float bits, copied by the gradient scan
  // before the update: the guard decides from this copy only, so every block
  // of every update kernel decides the same, whatever the update's own
  // blocks have since raised the live domain to.
  uint32_t snap[4];
  uint32_t pad[41];
  // Error bits of every push or update run in this workspace, OR-ed in as they
  // are found; the per-call clears of the block skip this word (it starts at
  // zero with the workspace and only eps_hip_status_history_word's user
  // clears it).  A caller that overlaps many pushes checks it once.
  uint32_t history;
};
static_assert(sizeof(Control) == 1024, "control block is 1 KiB");
constexpr uint32_t kHistoryWord = offsetof(Control, history) / 4;

// Error bits (a call that sets any of them wrote nothing, except a stall).
constexpr uint32_t kErrorBits = EPS_HIP_STATUS_BAD_INDEX | EPS_HIP_STATUS_NONFINITE_GRAD |
                                EPS_HIP_STATUS_REDUCE_OVERFLOW | EPS_HIP_STATUS_ADAM_OVERFLOW |
                                EPS_HIP_STATUS_BAD_SCALE;
constexpr uint32_t kHistoryBits = kErrorBits | EPS_HIP_STATUS_REJECTED | EPS_HIP_STATUS_STALLED;

enum Mode : uint32_t { kFused = 0, kChecked = 1, kReject = 2 };

// Adds status bits to the call's status word and its error bits to the
// workspace history.
__device__ __forceinline__ void ReportStatus(Control* ctrl, uint32_t bits) {
  if (!bits) return;
  atomicOr(&ctrl->status, bits);
  if (bits & kHistoryBits) atomicOr(&ctrl->history, bits & kHistoryBits);
}

// Bounds domain: kBoundSlots x {W, M, V, unused} as non-negative float bits.
struct Bounds { uint32_t v[kBoundSlots][4]; };

// A hot row: its sorted positions [start, end) and its key.
struct HotEntry { uint32_t start, end, key, pad; };

// Workspace layout of a push, for `n` occurrences.
struct PushLayout {
  uint64_t n, tiles, groups;
  uint64_t hist, look, group_look, keys_a, keys_b, vals_a, vals_b, refscale, sorted_rs, flags,
      ranks, block_sums, long_list, total;
  // Capacity of each hot-row list (any one may hold every hot row).
  constexpr uint64_t HotCapacity() const { return n / kLongRefs + 1; }
  constexpr explicit PushLayout(uint64_t occurrences)
      : n(occurrences), tiles(0), groups(0), hist(0), look(0), group_look(0), keys_a(0), keys_b(0), vals_a(0),
        vals_b(0), refscale(0), sorted_rs(0), flags(0), ranks(0), block_sums(0), long_list(0), total(0) {
    tiles = (n + kSortTile - 1) / kSortTile;
    groups = (tiles + kGroupTiles - 1) / kGroupTiles;
    auto align = [](uint64_t x) { return (x + 255) & ~uint64_t(255); };
    uint64_t at = sizeof(Control);
    hist = at; at = align(at + kHistCopies * kMaxPasses * kDigits * 4);
    look = at; at = align(at + kMaxPasses * tiles * kDigits * 4);
    group_look = at; at = align(at + kMaxPasses * groups * kDigits * 4);
    keys_a = at; at = align(at + n * 4);
    keys_b = at; at = align(at + n * 4);
    vals_a = at; at = align(at + n * 4);
    vals_b = at; at = align(at + n * 4);
    refscale = at; at = align(at + n * 8);
    sorted_rs = at; at = align(at + n * 8);
    flags = at; at = align(at + n * 4);
    ranks = at; at = align(at + n * 4);
    block_sums = at; at = align(at + ((n + 1023) / 1024 + 1) * 4);
    long_list = at; at = align(at + kXcds * kHotBuckets * HotCapacity() * sizeof(HotEntry));
    total = at;
  }
};

// ---- host-side error plumbing ----
void SetError(const std::string& message);
int Fail(int code, const std::string& message);
int Check(hipError_t e, const char* what);
#define EPS_HIP_TRY(expr) do { int rc_ = (expr); if (rc_) return rc_; } while (0)
#define EPS_HIP_LAUNCHED(what) EPS_HIP_TRY(::eps_hip::Check(hipGetLastError(), what))

inline hipStream_t AsStream(void* s) { return static_cast<hipStream_t>(s); }

// Fills count u32 words with value on the stream (a kernel, no memset node
// under graph capture), leaving word `keep` as it is.
int LaunchFill(uint32_t* target, uint32_t value, uint64_t count, hipStream_t stream,
               uint64_t keep = ~0ull);

// ---- device helpers ----
// Every buffer this library reads or writes is global memory (device memory,
// or pinned host memory through its mapped address).  Pointers that kernels
// fetch from LDS tables would otherwise compile to FLAT accesses, which also
// count against the LDS wait counter, so each LDS wait would stall on every
// outstanding global load; these accessors name the global address space.
#define EPS_GLOBAL __attribute__((address_space(1)))
typedef float EpsF4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float4 Load4(const float* p) {
  const EpsF4 v = *(const EPS_GLOBAL EpsF4*)(p);
  return make_float4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ void Store4(float* p, float4 v) {
  const EpsF4 x = {v.x, v.y, v.z, v.w};
  *(EPS_GLOBAL EpsF4*)(p) = x;
}
// Streaming forms for table state rows, which a push reads once and writes
// once: the nontemporal hint lets L2 evict them first, so the reused lines
// (gradient rows, sorted keys) stay resident while the state streams through.
__device__ __forceinline__ float4 Load4Stream(const float* p) {
  const EpsF4 v = __builtin_nontemporal_load((const EPS_GLOBAL EpsF4*)(p));
  return make_float4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ void Store4Stream(float* p, float4 v) {
  const EpsF4 x = {v.x, v.y, v.z, v.w};
  __builtin_nontemporal_store(x, (EPS_GLOBAL EpsF4*)(p));
}
__device__ __forceinline__ float LoadF(const float* p) { return *(const EPS_GLOBAL float*)(p); }
__device__ __forceinline__ void StoreF(float* p, float v) { *(EPS_GLOBAL float*)(p) = v; }
__device__ __forceinline__ uint32_t AbsBits(float x) { return __float_as_uint(x) & 0x7fffffffu; }
__device__ __forceinline__ bool Finite(float x) { return AbsBits(x) < 0x7f800000u; }

// Part (feature, span) a block belongs to, for launches that cover several
// parts ordered by their first block: the number of parts starting at or
// before this block, minus one.  One vector load and a ballot instead of a
// chain of dependent kernel-argument loads.
template <typename Part>
__device__ __forceinline__ uint32_t PartOf(const Part* parts, uint32_t count, uint32_t unit = blockIdx.x) {
  const uint32_t lane = threadIdx.x & (kWave - 1);
  const uint32_t begin = lane < count ? parts[lane].block_begin : 0xffffffffu;
  return uint32_t(__popcll(__ballot(begin <= unit))) - 1u;
}

// Maximum over the lanes of a wavefront (DPP/permute lowering by the compiler).
__device__ __forceinline__ uint32_t WaveMax(uint32_t x) {
#pragma unroll
  for (int offset = 32; offset > 0; offset >>= 1) x = max(x, (uint32_t)__shfl_xor((int)x, offset));
  return x;
}

// First index q in [from, limit) with keys[q] != key, or limit (keys sorted):
// exponential then binary search, so long runs cost O(log run).
__device__ inline uint32_t SegmentEndSearch(const uint32_t* keys, uint32_t from, uint32_t limit,
                                            uint32_t key) {
  if (from >= limit || keys[from] != key) return from;
  uint32_t lo = from, step = 1, hi;
  for (;;) {
    const uint32_t q = lo + step;
    if (q >= limit || q < lo) { hi = limit; break; }
    if (keys[q] != key) { hi = q; break; }
    lo = q;
    step <<= 1;
  }
  while (hi - lo > 1) {
    const uint32_t mid = lo + ((hi - lo) >> 1);
    if (keys[mid] == key) lo = mid; else hi = mid;
  }
  return hi;
}

// BoundWeight (src/common/optimizer_bounds.hpp:14-18) written as std::clamp so
// signed zeros match the CPU exactly.
__device__ __forceinline__ float Clamp(float v, float lo, float hi) {
  return v < lo ? lo : (hi < v ? hi : v);
}

}  // namespace eps_hip
