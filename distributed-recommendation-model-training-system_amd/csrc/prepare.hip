// prepare.hip -- device-side dedup of pushed occurrences by row.
//
// The reference dedups on the host with a hash map in first-occurrence order
// (PrepareFeature, src/access/batch_access.cpp:32-36; ReduceGradients, :73-93)
// and ships either reduced rows or a host-built CSR to the device
// (BuildCompactGradients, src/access/compact_gradients.cpp:43-72).  Here the
// grouping is a stable LSD radix sort of 32-bit keys (key index << row_bits |
// slot) carrying the occurrence index, so equal rows end up adjacent in
// occurrence order -- exactly the CSR order of the reference's references
// (repeats kept, (feature, bag, position) order).
//
//   keygen : one pass over the occurrences -> key, occurrence index, packed
//            (gradient row | scale) reference word, all-pass digit histograms,
//            per-class valid counts, max |scale|.
//   passes : onesweep (single pass per digit): per-tile stable ranking with
//            wavefront ballots, two-level decoupled look-back (over groups of
//            tiles) for the digit prefix, LDS-staged scatter so each digit run is written
//            contiguously.  The last pass also scatters the reference words.
//   unique : first-occurrence ranks (PrepareFeature's unique order) from a
//            head-flag scan in occurrence space.
#include "prepare.hpp"

#include <algorithm>

namespace eps_hip {

namespace {

constexpr uint32_t kFlagAggregate = 1u << 30;
constexpr uint32_t kFlagInclusive = 2u << 30;
constexpr uint32_t kValueMask = (1u << 30) - 1;
constexpr uint32_t kLookWindow = 16;  // predecessor groups read per look-back round
constexpr uint32_t kStageBags = 2048;   // bag offsets a keygen block stages in LDS

struct PrepFeature {
  const uint64_t* indices;
  const uint64_t* offsets;
  const uint64_t* lengths;
  const float* weights;
  uint64_t occ_begin, occurrences, bags, table_rows;
  uint32_t key_index, pooling, block_begin, feature;
};
struct PrepArgs {
  PrepFeature f[EPS_HIP_MAX_FEATURES];
  uint32_t count, row_bits, sentinel, passes;
  uint32_t shift[kMaxPasses], bits[kMaxPasses];
  Control* ctrl;
  uint32_t* hist;
  uint32_t* keys;
  uint32_t* vals;
  uint64_t* refscale;  // reference words with their scales (8 bytes), or
  uint32_t* refs;      // without (4 bytes: no weighted-sum feature; the scale is derived)
  // Words that keygen's blocks clear (the group look-back flags of the
  // passes, which only the passes after keygen read): one fill launch fewer.
  uint32_t* zero;
  uint64_t zero_words;
};
static_assert(sizeof(PrepArgs) <= 4096, "keygen arguments fit the kernel-argument segment");

// What the last pass needs to put each reference word's scale back (pushes
// with no weighted-sum feature sort 4-byte words without it): the mean
// features and their valid lengths.  The scale is then exactly what keygen
// computes: 1.0f / (float)len for a mean bag of nonzero length, else 1.0f.
struct ScaleArgs {
  const uint64_t* lengths[EPS_HIP_MAX_FEATURES];
  uint32_t mean_mask;  // bit f: feature f is mean-pooled
};

__global__ void __launch_bounds__(kBlock) KeygenKernel(PrepArgs args) {
  const PrepFeature f = args.f[PartOf(args.f, args.count)];
  __shared__ uint32_t s_hist[kMaxPasses][kDigits];
  __shared__ uint32_t s_misc[2];  // [0] bad, [1] max scale
  __shared__ uint64_t s_off[kStageBags];  // offsets[b0 .. b0 + staged)
  __shared__ uint64_t s_b0;
  for (uint64_t i = uint64_t(blockIdx.x) * kBlock + threadIdx.x; i < args.zero_words;
       i += uint64_t(gridDim.x) * kBlock)
    args.zero[i] = 0;
  for (uint32_t i = threadIdx.x; i < kMaxPasses * kDigits; i += kBlock) (&s_hist[0][0])[i] = 0;
  if (threadIdx.x < 2) s_misc[threadIdx.x] = 0;

  const uint64_t local0 = uint64_t(blockIdx.x - f.block_begin) * (kBlock * kKeygenItems);
  uint32_t scale_max = 0;
  bool bad = false;
  // The thread's occurrences are independent: their slot loads, bag searches
  // and scale loads proceed interleaved, so each dependent step has all of
  // them in flight instead of one.
  uint64_t li[kKeygenItems], slot[kKeygenItems], lo[kKeygenItems];
  bool in[kKeygenItems];
#pragma unroll
  for (uint32_t k = 0; k < kKeygenItems; ++k) {
    li[k] = local0 + k * kBlock + threadIdx.x;
    in[k] = li[k] < f.occurrences;
    slot[k] = in[k] ? f.indices[li[k]] : kHole;
    lo[k] = 0;  // bag of the occurrence: largest b < bags with offsets[b] <= li
  }
  if (f.pooling != EPS_HIP_POOL_SEQUENCE) {
    // Bag of each occurrence: the largest b < bags with offsets[b] <= li.
    // The block's occurrences are consecutive, so wavefront 0 first finds the
    // bag b0 of the block's first occurrence with a 64-way search (each round
    // probes 64 evenly spaced offsets at once and keeps the segment the ballot
    // points at: two rounds for 4096 bags), the block then stages
    // offsets[b0 ..] in LDS, and each occurrence is searched there.
    const uint64_t first = local0, last = min(local0 + kBlock * kKeygenItems, f.occurrences) - 1;
    if (threadIdx.x < kWave) {
      const uint32_t lane = threadIdx.x;
      uint64_t base = 0, len = f.bags;  // answer in [base, base + len); offsets[base] <= first or base == 0
      while (len > 1) {
        const uint64_t step = (len + kWave - 1) / kWave;
        const uint64_t q = uint64_t(lane) * step;
        const bool probe = q < len && f.offsets[base + q] <= first;
        const uint32_t count = uint32_t(__popcll(__ballot(probe)));
        const uint64_t keep = count ? count - 1 : 0;
        base += keep * step;
        len = min(step, len - keep * step);
      }
      if (lane == 0) s_b0 = base;
    }
    __syncthreads();
    const uint64_t b0 = s_b0;
    const uint32_t staged = uint32_t(min<uint64_t>(kStageBags, f.bags + 1 - b0));
    for (uint32_t i = threadIdx.x; i < staged; i += kBlock) s_off[i] = f.offsets[b0 + i];
    __syncthreads();
    // Covered when the staged offsets reach past the block's last occurrence
    // (or reach offsets[bags], which is past every occurrence); else (runs of
    // empty bags longer than the stage) fall back to searching global memory.
    if (b0 + staged == f.bags + 1 || s_off[staged - 1] > last) {
      uint32_t r[kKeygenItems];
#pragma unroll
      for (uint32_t k = 0; k < kKeygenItems; ++k) r[k] = 0;
      // Answer in [0, staged - 1): offsets[b0 + staged - 1] > last unless it is offsets[bags].
      for (uint32_t len = staged - 1; len > 1;) {
        const uint32_t half = len >> 1;
#pragma unroll
        for (uint32_t k = 0; k < kKeygenItems; ++k) r[k] = s_off[r[k] + half] <= li[k] ? r[k] + half : r[k];
        len -= half;
      }
#pragma unroll
      for (uint32_t k = 0; k < kKeygenItems; ++k) lo[k] = b0 + r[k];
    } else {
      // Branch-free binary search with a trip count that is uniform over the
      // block: each step issues all of the thread's offset loads before it
      // waits on them.  The probe lo + half stays below lo + len <= bags.
      for (uint64_t len = f.bags; len > 1;) {
        const uint64_t half = len >> 1;
        uint64_t probe[kKeygenItems];
#pragma unroll
        for (uint32_t k = 0; k < kKeygenItems; ++k) probe[k] = f.offsets[lo[k] + half];
#pragma unroll
        for (uint32_t k = 0; k < kKeygenItems; ++k) lo[k] = probe[k] <= li[k] ? lo[k] + half : lo[k];
        len -= half;
      }
    }
  } else {
    __syncthreads();
  }
  // Per-occurrence scale, loaded for all items before any is used (the pooling
  // mode is uniform over the block; indices are clamped into range).
  float scale[kKeygenItems];
#pragma unroll
  for (uint32_t k = 0; k < kKeygenItems; ++k) scale[k] = 1.0f;
  if (f.pooling == EPS_HIP_POOL_MEAN) {
    uint64_t len[kKeygenItems];
#pragma unroll
    for (uint32_t k = 0; k < kKeygenItems; ++k) len[k] = f.lengths[lo[k]];
#pragma unroll
    for (uint32_t k = 0; k < kKeygenItems; ++k)
      if (len[k]) scale[k] = 1.0f / (float)len[k];  // batch_access.cpp:79-80
  } else if (f.pooling == EPS_HIP_POOL_WEIGHTED_SUM) {
#pragma unroll
    for (uint32_t k = 0; k < kKeygenItems; ++k)
      scale[k] = f.weights[in[k] ? li[k] : f.occurrences - 1];
  }
#pragma unroll
  for (uint32_t k = 0; k < kKeygenItems; ++k) {
    if (!in[k]) continue;
    const uint64_t gi = f.occ_begin + li[k];
    uint64_t s = slot[k];
    if (s != kHole && s >= f.table_rows) { bad = true; s = kHole; }
    uint32_t key = args.sentinel;
    if (s != kHole) key = (f.key_index << args.row_bits) | uint32_t(s);
    const uint64_t row = f.pooling == EPS_HIP_POOL_SEQUENCE ? li[k] : lo[k];
    if (s != kHole) scale_max = max(scale_max, AbsBits(scale[k]));
    args.keys[gi] = key;
    if (args.vals) args.vals[gi] = uint32_t(gi);
    const uint32_t ref = (f.feature << kRefRowBits) | uint32_t(row);
    if (args.refs) args.refs[gi] = ref;
    else args.refscale[gi] = (uint64_t(__float_as_uint(scale[k])) << 32) | ref;
    for (uint32_t p = 0; p < args.passes; ++p)
      atomicAdd(&s_hist[p][(key >> args.shift[p]) & ((1u << args.bits[p]) - 1)], 1u);
  }
  if (bad) s_misc[0] = 1;
  // Only scales above 1.0 matter to the guard (it bounds with max(1, |scale|)),
  // so sum and mean pooling never reach the atomics below.
  scale_max = WaveMax(scale_max);
  if ((threadIdx.x & (kWave - 1)) == 0 && scale_max > 0x3f800000u) atomicMax(&s_misc[1], scale_max);
  __syncthreads();
  // The block's histogram goes to one of kHistCopies copies (round robin);
  // the radix passes add the copies up.
  uint32_t* hist = args.hist + (blockIdx.x % kHistCopies) * (kMaxPasses * kDigits);
  for (uint32_t i = threadIdx.x; i < args.passes * kDigits; i += kBlock) {
    const uint32_t c = (&s_hist[0][0])[i];
    if (c) atomicAdd(hist + i, c);
  }
  if (threadIdx.x == 0) {
    if (s_misc[0]) atomicOr(&args.ctrl->prep_status, EPS_HIP_STATUS_BAD_INDEX);
    if (s_misc[1]) atomicMax(&args.ctrl->scale_slots[blockIdx.x % kSrcSlots], s_misc[1]);
  }
}

// Exclusive scan of one value per thread over a 256-thread block.
__device__ __forceinline__ uint32_t BlockExclusiveScan(uint32_t x, uint32_t* s_wave) {
  const uint32_t lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  uint32_t inc = x;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t y = __shfl_up(inc, o);
    if (lane >= uint32_t(o)) inc += y;
  }
  if (lane == kWave - 1) s_wave[wave] = inc;
  __syncthreads();
  uint32_t before = 0;
  for (uint32_t w = 0; w < wave; ++w) before += s_wave[w];
  __syncthreads();
  return before + inc - x;
}

// kVals: the occurrence indices travel with the keys (for eps_hip_unique and
// eps_hip_reduce, which map sorted positions back to occurrences); a push
// needs only the keys and reference words.  kWords: the reference words are
// 8 bytes with their scales (kWide), 4 bytes without (kNarrow), or 4 bytes
// in and 8 bytes out (kWiden, the last pass of a sort of 4-byte words, which
// puts each word's scale back from ScaleArgs).
enum WordForm : int { kWide = 0, kNarrow = 1, kWiden = 2 };
template <int kWords> struct WordTypes;
template <> struct WordTypes<kWide> { typedef uint64_t In; typedef uint64_t Out; };
template <> struct WordTypes<kNarrow> { typedef uint32_t In; typedef uint32_t Out; };
template <> struct WordTypes<kWiden> { typedef uint32_t In; typedef uint64_t Out; };

template <bool kVals, int kWords>
__global__ void __launch_bounds__(kBlock) RadixPassKernel(
    const uint32_t* __restrict__ keys_in, const uint32_t* __restrict__ vals_in,
    uint32_t* __restrict__ keys_out, uint32_t* __restrict__ vals_out,
    const typename WordTypes<kWords>::In* __restrict__ rs_in, typename WordTypes<kWords>::Out* __restrict__ rs_out,
    uint32_t n, uint32_t shift, uint32_t bits, const uint32_t* __restrict__ hist, uint32_t* look,
    uint32_t* group_look, uint32_t tiles, uint32_t* tile_counter, ScaleArgs sc) {
  typedef typename WordTypes<kWords>::In InWord;
  __shared__ uint32_t s_tile;
  __shared__ uint32_t s_wcount[4][kDigits];
  __shared__ uint32_t s_tile_start[kDigits];
  __shared__ uint32_t s_global[kDigits];
  __shared__ uint32_t s_scan[4];
  __shared__ uint32_t s_keys[kSortTile];
  __shared__ uint32_t s_vals[kVals ? kSortTile : 1];
  __shared__ InWord s_rs[kSortTile];

  const uint32_t t = threadIdx.x, lane = t & (kWave - 1), wave = t / kWave;
  if (t == 0) s_tile = atomicAdd(tile_counter, 1u);
  for (uint32_t i = t; i < 4 * kDigits; i += kBlock) (&s_wcount[0][0])[i] = 0;
  __syncthreads();
  const uint32_t tile = s_tile;
  // This thread's digits are 2t and 2t+1; their global counts (the sum of
  // the keygen copies) are loaded early.
  uint32_t digit_count[kDigitsPerThread] = {0, 0};
#pragma unroll
  for (uint32_t c = 0; c < kHistCopies; ++c)
#pragma unroll
    for (uint32_t j = 0; j < kDigitsPerThread; ++j)
      digit_count[j] += hist[c * (kMaxPasses * kDigits) + kDigitsPerThread * t + j];
  const uint32_t mask = (1u << bits) - 1;
  const uint32_t base = tile * kSortTile + wave * (kSortTile / 4);
  uint32_t key[kSortItems], val[kSortItems], rank[kSortItems];
  InWord rs[kSortItems];
#pragma unroll
  for (uint32_t i = 0; i < kSortItems; ++i) {
    const uint32_t p = base + i * kWave + lane;
    key[i] = p < n ? keys_in[p] : 0u;
    val[i] = kVals && p < n ? vals_in[p] : 0u;
    rs[i] = p < n ? rs_in[p] : InWord(0);
  }
  const uint64_t lt_mask = (1ull << lane) - 1;
#pragma unroll
  for (uint32_t i = 0; i < kSortItems; ++i) {
    const uint32_t p = base + i * kWave + lane;
    const bool valid = p < n;
    const uint32_t digit = (key[i] >> shift) & mask;
    uint64_t match = __ballot(valid);
    for (uint32_t b = 0; b < bits; ++b) {
      const bool bit = (digit >> b) & 1u;
      const uint64_t ones = __ballot(bit);
      match &= bit ? ones : ~ones;
    }
    rank[i] = 0;
    if (valid) {
      const uint32_t before = s_wcount[wave][digit];
      rank[i] = before + uint32_t(__popcll(match & lt_mask));
      if (lane == uint32_t(__ffsll((unsigned long long)match) - 1))
        s_wcount[wave][digit] = before + uint32_t(__popcll(match));
    }
  }
  __syncthreads();
  // Per digit (two per thread): wave prefixes, tile total, look-back.
  uint32_t total[kDigitsPerThread], exclusive[kDigitsPerThread];
#pragma unroll
  for (uint32_t j = 0; j < kDigitsPerThread; ++j) {
    const uint32_t d = kDigitsPerThread * t + j;
    total[j] = 0;
    exclusive[j] = 0;
#pragma unroll
    for (uint32_t w = 0; w < 4; ++w) {
      const uint32_t c = s_wcount[w][d];
      s_wcount[w][d] = total[j];
      total[j] += c;
    }
  }
  // Two-level look-back.  Tiles form groups of kGroupTiles; every tile
  // publishes its digit counts.  A tile's exclusive prefix is the counts of
  // the tiles before it in its group plus the prefix of the groups before
  // its group.  The group's last tile publishes the group total, then (after
  // its own walk) the group's inclusive prefix.  The walk over groups is
  // windowed and stops at the first inclusive prefix, as a tile-level
  // look-back would, but the chain runs through groups, not tiles.  A tile
  // waits only on tiles claimed before it (the tile counter hands tiles out in
  // order), so the waits always end.
  const uint32_t group = tile / kGroupTiles, first = group * kGroupTiles;
  const bool leader = tile + 1 == min(first + kGroupTiles, tiles);
  uint32_t* mine = look + uint64_t(tile) * kDigits + kDigitsPerThread * t;
#pragma unroll
  for (uint32_t j = 0; j < kDigitsPerThread; ++j)
    __hip_atomic_store(mine + j, kFlagAggregate | total[j], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  // Counts of the tiles before this one in its group (all published or about to be).
  uint32_t within[kDigitsPerThread] = {0, 0};
  {
    uint32_t missing = (1u << (tile - first)) - 1;  // bit w: tile first + w still to add
    while (missing) {
      uint32_t v[kDigitsPerThread][kGroupTiles];
#pragma unroll
      for (uint32_t w = 0; w < kGroupTiles; ++w)
#pragma unroll
        for (uint32_t j = 0; j < kDigitsPerThread; ++j)
          v[j][w] = (missing >> w) & 1u
                        ? __hip_atomic_load(look + uint64_t(first + w) * kDigits + kDigitsPerThread * t + j,
                                            __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                        : 0u;
#pragma unroll
      for (uint32_t w = 0; w < kGroupTiles; ++w) {
        if (!((missing >> w) & 1u) || !(v[0][w] & ~kValueMask) || !(v[1][w] & ~kValueMask)) continue;
#pragma unroll
        for (uint32_t j = 0; j < kDigitsPerThread; ++j) within[j] += v[j][w] & kValueMask;
        missing &= ~(1u << w);
      }
    }
  }
  uint32_t* group_mine = group_look + uint64_t(group) * kDigits + kDigitsPerThread * t;
  if (leader)
#pragma unroll
    for (uint32_t j = 0; j < kDigitsPerThread; ++j)
      __hip_atomic_store(group_mine + j, (group == 0 ? kFlagInclusive : kFlagAggregate) | (within[j] + total[j]),
                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  // Windowed walk over the groups before this one: each round reads the
  // next kLookWindow predecessors of every unfinished digit at once and adds
  // their counts, nearest first, up to the first inclusive prefix (done) or
  // the first group that has not published yet (read again from there).
  // Group 0 always publishes an inclusive prefix, so each walk ends at or
  // before it; reads before group 0 are never issued.
  int64_t next[kDigitsPerThread];
  bool done[kDigitsPerThread];
#pragma unroll
  for (uint32_t j = 0; j < kDigitsPerThread; ++j) { next[j] = int64_t(group) - 1; done[j] = group == 0; }
  while (!done[0] || !done[1]) {
    uint32_t v[kDigitsPerThread][kLookWindow];
#pragma unroll
    for (uint32_t j = 0; j < kDigitsPerThread; ++j)
#pragma unroll
      for (uint32_t w = 0; w < kLookWindow; ++w) {
        const int64_t q = next[j] - int64_t(w);
        v[j][w] = (!done[j] && q >= 0)
                      ? __hip_atomic_load(group_look + uint64_t(q) * kDigits + kDigitsPerThread * t + j,
                                          __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                      : kFlagInclusive;
      }
#pragma unroll
    for (uint32_t j = 0; j < kDigitsPerThread; ++j) {
      if (done[j]) continue;
      bool stop = false;
      uint32_t taken = 0;
#pragma unroll
      for (uint32_t w = 0; w < kLookWindow; ++w) {
        const uint32_t flag = v[j][w] & ~kValueMask;
        if (!stop) {
          if (flag == 0) {
            stop = true;  // not published yet
          } else {
            exclusive[j] += v[j][w] & kValueMask;
            ++taken;
            if (flag == kFlagInclusive) stop = done[j] = true;
          }
        }
      }
      next[j] -= int64_t(taken);
    }
  }
  if (leader && group != 0)
#pragma unroll
    for (uint32_t j = 0; j < kDigitsPerThread; ++j)
      __hip_atomic_store(group_mine + j, kFlagInclusive | (exclusive[j] + within[j] + total[j]),
                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
  for (uint32_t j = 0; j < kDigitsPerThread; ++j) exclusive[j] += within[j];
  // Exclusive scans in digit order: thread t's pair (2t, 2t+1) is one scan item.
  const uint32_t digit_base = BlockExclusiveScan(digit_count[0] + digit_count[1], s_scan);
  const uint32_t tile_start = BlockExclusiveScan(total[0] + total[1], s_scan);
  s_tile_start[2 * t] = tile_start;
  s_tile_start[2 * t + 1] = tile_start + total[0];
  s_global[2 * t] = digit_base + exclusive[0];
  s_global[2 * t + 1] = digit_base + digit_count[0] + exclusive[1];
  __syncthreads();
#pragma unroll
  for (uint32_t i = 0; i < kSortItems; ++i) {
    const uint32_t p = base + i * kWave + lane;
    if (p < n) {
      const uint32_t digit = (key[i] >> shift) & mask;
      const uint32_t at = s_tile_start[digit] + s_wcount[wave][digit] + rank[i];
      s_keys[at] = key[i];
      if (kVals) s_vals[at] = val[i];
      s_rs[at] = rs[i];
    }
  }
  __syncthreads();
  // Scatter of the digit-sorted tile: all LDS reads, then the stores.  The
  // reference words travel with their keys through every pass, so the last
  // pass needs no gather by occurrence index.  Entries past the tile's end
  // read stale LDS (in bounds) and are not stored.
  const uint32_t tile_n = min(kSortTile, n - tile * kSortTile);
  uint32_t dest[kSortItems];
#pragma unroll
  for (uint32_t i = 0; i < kSortItems; ++i) {
    const uint32_t q = i * kBlock + t;
    key[i] = s_keys[q];
    if (kVals) val[i] = s_vals[q];
    rs[i] = s_rs[q];
    const uint32_t digit = (key[i] >> shift) & mask;
    dest[i] = s_global[digit] + (q - s_tile_start[digit]);
  }
  if (kWords == kWiden) {
    // Each word's scale: the valid length of a mean feature's bag (all
    // loaded before any is used), as keygen computed it.
    uint64_t len[kSortItems];
#pragma unroll
    for (uint32_t i = 0; i < kSortItems; ++i) {
      const uint32_t feature = uint32_t(rs[i]) >> kRefRowBits;
      const bool mean = i * kBlock + t < tile_n && ((sc.mean_mask >> feature) & 1u);
      len[i] = mean ? sc.lengths[feature][uint32_t(rs[i]) & ((1u << kRefRowBits) - 1u)] : 0ull;
    }
#pragma unroll
    for (uint32_t i = 0; i < kSortItems; ++i) {
      if (i * kBlock + t < tile_n) {
        const float scale = len[i] ? 1.0f / (float)len[i] : 1.0f;  // batch_access.cpp:79-80
        keys_out[dest[i]] = key[i];
        if (kVals) vals_out[dest[i]] = val[i];
        rs_out[dest[i]] = typename WordTypes<kWords>::Out((uint64_t(__float_as_uint(scale)) << 32) | uint32_t(rs[i]));
      }
    }
    return;
  }
#pragma unroll
  for (uint32_t i = 0; i < kSortItems; ++i) {
    if (i * kBlock + t < tile_n) {
      keys_out[dest[i]] = key[i];
      if (kVals) vals_out[dest[i]] = val[i];
      rs_out[dest[i]] = typename WordTypes<kWords>::Out(rs[i]);
    }
  }
}

// ---- first-occurrence ranking ----
__global__ void HeadFlagKernel(const uint32_t* keys, const uint32_t* vals, const Control* ctrl,
                               uint32_t* flags, uint32_t n) {
  const uint32_t valid = ctrl->valid_count;
  for (uint32_t p = blockIdx.x * blockDim.x + threadIdx.x; p < n && p < valid;
       p += blockDim.x * gridDim.x)
    if (p == 0 || keys[p] != keys[p - 1]) flags[vals[p]] = 1;
}

__global__ void ScanBlockSumsKernel(const uint32_t* flags, uint32_t* block_sums, uint32_t n) {
  __shared__ uint32_t s_wave[4];
  const uint32_t b = blockIdx.x;
  uint32_t sum = 0;
  for (uint32_t k = 0; k < 4; ++k) {
    const uint32_t i = b * 1024 + k * kBlock + threadIdx.x;
    if (i < n) sum += flags[i];
  }
  const uint32_t lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  for (int o = 32; o > 0; o >>= 1) sum += __shfl_xor(sum, o);
  if (lane == 0) s_wave[wave] = sum;
  __syncthreads();
  if (threadIdx.x == 0) block_sums[b] = s_wave[0] + s_wave[1] + s_wave[2] + s_wave[3];
}

__global__ void ScanTopKernel(uint32_t* block_sums, uint32_t blocks, Control* ctrl,
                              uint64_t* unique_count) {
  __shared__ uint32_t s_scan[4];
  __shared__ uint32_t s_carry;
  if (threadIdx.x == 0) s_carry = 0;
  __syncthreads();
  for (uint32_t start = 0; start < blocks; start += kBlock) {
    const uint32_t i = start + threadIdx.x;
    const uint32_t x = i < blocks ? block_sums[i] : 0;
    const uint32_t ex = BlockExclusiveScan(x, s_scan);
    const uint32_t carry = s_carry;
    if (i < blocks) block_sums[i] = carry + ex;
    __syncthreads();
    if (threadIdx.x == kBlock - 1) s_carry = carry + ex + x;
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    ctrl->unique_count = s_carry;
    if (unique_count) *unique_count = s_carry;
  }
}

__global__ void ScanApplyKernel(const uint32_t* flags, const uint32_t* block_sums, uint32_t* ranks,
                                uint32_t n) {
  __shared__ uint32_t s_scan[4];
  __shared__ uint32_t s_carry;
  const uint32_t b = blockIdx.x;
  if (threadIdx.x == 0) s_carry = block_sums[b];
  __syncthreads();
  for (uint32_t k = 0; k < 4; ++k) {
    const uint32_t i = b * 1024 + k * kBlock + threadIdx.x;
    const uint32_t x = i < n ? flags[i] : 0;
    const uint32_t ex = BlockExclusiveScan(x, s_scan);
    const uint32_t carry = s_carry;
    if (i < n) ranks[i] = carry + ex;
    __syncthreads();
    if (threadIdx.x == kBlock - 1) s_carry = carry + ex + x;
    __syncthreads();
  }
}

// ---- hot rows: segments of more than kLongRefs references ----
// Keys are sorted, so a segment that starts at p has more than kLongRefs
// references exactly when keys[p + kLongRefs] == keys[p]: one test per
// position, no scan.  Only vector dimension classes are listed (the generic
// class keeps its own kernel).  The list order is irrelevant: rows are
// independent.
struct HotArgs {
  const uint32_t* keys;
  HotEntry* hot;
  Control* ctrl;
  uint32_t n, row_bits, capacity, sentinel;
  uint32_t class_key[kClasses + 1];  // first table key index of each class (+ table count)
};

// Dimension class of a sorted key; the sentinel (rows not on this device; it
// is above every valid key, so it sorts last) is class kClasses.
__device__ __forceinline__ uint32_t ClassOfKey(const HotArgs& a, uint32_t key) {
  if (key == a.sentinel) return kClasses;
  const uint32_t ki = key >> a.row_bits;
  uint32_t c = 0;
#pragma unroll
  for (uint32_t k = 1; k <= kClasses; ++k) c += ki >= a.class_key[k];
  return c;
}

// One thread per sorted position p (and one for p == n):
//  * class boundaries: class_start[c] = first position whose class is >= c,
//    written by the one position where the class steps over c (the keys are
//    sorted and key indices are ordered by class); class_start[kClasses] is
//    the number of valid occurrences;
//  * hot rows: a vector-class row with more than kLongRefs references (its
//    positions and key) is appended, by the thread at its first position, to
//    one of the lists of the XCD that owns that eighth of the positions (the
//    update kernels split their work the same way); the row's length picks
//    the list (eight ranges, from 65,536 or more references down), so the
//    hot-row kernel can deal the longest rows out first.
__global__ void __launch_bounds__(kBlock) HotListKernel(HotArgs a) {
  const uint32_t p = blockIdx.x * kBlock + threadIdx.x;
  if (p > a.n) return;
  const uint32_t key = p < a.n ? a.keys[p] : 0u;
  const uint32_t cls = p < a.n ? ClassOfKey(a, key) : kClasses;
  const uint32_t pkey = p > 0 ? a.keys[p - 1] : 0u;
  const bool first = p == 0 || pkey != key;
  // Classes prev..cls start at p.
  const uint32_t prev = p == 0 ? 0u : ClassOfKey(a, pkey) + 1u;
  for (uint32_t c = prev; c <= cls; ++c) {
    a.ctrl->class_start[c] = p;
    if (c == kClasses) a.ctrl->valid_count = p;
  }
  if (p >= a.n || cls + 1 >= kClasses || !first) return;
  if (p + kLongRefs >= a.n || a.keys[p + kLongRefs] != key) return;
  const uint32_t end = SegmentEndSearch(a.keys, p + kLongRefs, a.n, key), refs = end - p;
  // Lists by length, longest first: >= 65536, 16384, 4096, 2048, 1024, 512, 256, fewer.
  const uint32_t bucket = refs >= 65536 ? 0u : refs >= 16384 ? 1u : refs >= 4096 ? 2u : refs >= 2048 ? 3u :
                          refs >= 1024 ? 4u : refs >= 512 ? 5u : refs >= 256 ? 6u : 7u;
  const uint32_t list = uint32_t(uint64_t(p) * kXcds / a.n) * kHotBuckets + bucket;
  // Sorted keys give each hot row one first position, so a list never holds
  // more than n / 129 entries; the bound keeps the write inside the list
  // whatever the keys (the readers clamp the counts to the capacity too).
  const uint32_t at = atomicAdd(&a.ctrl->long_count[list], 1u);
  if (at < a.capacity) a.hot[uint64_t(list) * a.capacity + at] = HotEntry{p, end, key, 0u};
}

struct UniqueArgs {
  uint32_t table_of_key[EPS_HIP_MAX_TABLES];
};

__global__ void UniqueWriteKernel(const uint32_t* keys, const uint32_t* vals, const uint32_t* ranks,
                                  const Control* ctrl, uint32_t n, uint32_t row_bits,
                                  UniqueArgs args, uint64_t* unique_slots, uint32_t* unique_tables,
                                  uint64_t* occurrence_to_unique) {
  const uint32_t valid = ctrl->valid_count;
  __shared__ uint32_t s_table[EPS_HIP_MAX_TABLES];
#pragma unroll
  for (uint32_t i = 0; i < EPS_HIP_MAX_TABLES; ++i)
    if (threadIdx.x == i) s_table[i] = args.table_of_key[i];
  __syncthreads();
  for (uint32_t p = blockIdx.x * blockDim.x + threadIdx.x; p < n && p < valid;
       p += blockDim.x * gridDim.x) {
    const uint32_t key = keys[p];
    uint32_t lo = 0, hi = p;  // first index with this key (lower bound) in [lo, hi]
    while (lo < hi) {
      const uint32_t mid = (lo + hi) >> 1;
      if (keys[mid] < key) lo = mid + 1; else hi = mid;
    }
    const uint32_t u = ranks[vals[lo]];
    occurrence_to_unique[vals[p]] = u;
    if (lo == p) {
      unique_slots[u] = key & ((1u << row_bits) - 1);
      unique_tables[u] = s_table[key >> row_bits];
    }
  }
}

unsigned Grid(uint64_t n, unsigned cap) {
  const uint64_t b = (n + kBlock - 1) / kBlock;
  return unsigned(std::max<uint64_t>(1, std::min<uint64_t>(b, cap)));
}

uint32_t BitLength(uint64_t x) {
  uint32_t b = 0;
  while (x) { ++b; x >>= 1; }
  return b;
}

}  // namespace

int PlanPush(const eps_hip_table* tables, uint32_t table_count,
             const eps_hip_push_feature* features, uint32_t feature_count, PushPlan& plan) {
  if (!tables || table_count == 0 || table_count > EPS_HIP_MAX_TABLES)
    return Fail(EPS_HIP_INVALID_ARGUMENT, "push needs 1..32 tables");
  if (!features || feature_count == 0 || feature_count > EPS_HIP_MAX_FEATURES)
    return Fail(EPS_HIP_INVALID_ARGUMENT, "push needs 1..32 features");
  uint64_t max_rows = 1;
  for (uint32_t t = 0; t < table_count; ++t) {
    if (!tables[t].state || tables[t].dim == 0 || tables[t].dim > 65536)
      return Fail(EPS_HIP_INVALID_ARGUMENT, "invalid push table");
    if (reinterpret_cast<uintptr_t>(tables[t].state) % 16)
      return Fail(EPS_HIP_INVALID_ARGUMENT, "table state must be 16-byte aligned");
    max_rows = std::max<uint64_t>(max_rows, tables[t].rows);
  }
  plan.row_bits = std::max<uint32_t>(1, BitLength(max_rows - 1));
  // Table key indices ordered by dimension class, so each class is one
  // contiguous range of the sorted keys (tables of a class in call order).
  uint32_t keyed = 0;
  for (uint32_t c = 0; c < kClasses; ++c)
    for (uint32_t t = 0; t < table_count; ++t)
      if (DimClass(tables[t].dim) == c) plan.table_of_key[keyed++] = t;
  for (uint32_t i = 0; i < table_count; ++i) plan.key_index[plan.table_of_key[i]] = i;
  const auto& order = plan.table_of_key;
  for (uint32_t c = 0; c <= kClasses; ++c) {
    uint32_t k = 0;
    while (k < table_count && DimClass(tables[order[k]].dim) < c) ++k;
    plan.class_start[c] = k;
  }
  const uint64_t max_valid = (uint64_t(table_count - 1) << plan.row_bits) | (max_rows - 1);
  plan.key_bits = BitLength(max_valid + 1);
  if (plan.key_bits > 32) return Fail(EPS_HIP_CAPACITY_EXCEEDED, "table rows exceed 32-bit sort keys");
  plan.passes = (plan.key_bits + kRadixBits - 1) / kRadixBits;
  if (plan.passes > kMaxPasses) return Fail(EPS_HIP_CAPACITY_EXCEEDED, "sort keys need too many passes");
  uint32_t at = 0;
  for (uint32_t p = 0; p < plan.passes; ++p) {
    const uint32_t remaining = plan.key_bits - at, left = plan.passes - p;
    plan.bits[p] = (remaining + left - 1) / left;
    plan.shift[p] = at;
    at += plan.bits[p];
  }
  plan.occurrences = 0;
  plan.class_occurrences.fill(0);
  for (uint32_t i = 0; i < feature_count; ++i) {
    const auto& f = features[i];
    if (f.table >= table_count || f.pooling > EPS_HIP_POOL_WEIGHTED_SUM)
      return Fail(EPS_HIP_INVALID_ARGUMENT, "invalid push feature");
    if (f.occurrences && !f.indices) return Fail(EPS_HIP_INVALID_ARGUMENT, "null feature indices");
    if (f.pooling != EPS_HIP_POOL_SEQUENCE && (!f.offsets || (f.pooling == EPS_HIP_POOL_MEAN && !f.valid_lengths)))
      return Fail(EPS_HIP_INVALID_ARGUMENT, "pooled feature needs offsets (and lengths for mean)");
    if (f.pooling != EPS_HIP_POOL_SEQUENCE && f.occurrences && !f.bags)
      return Fail(EPS_HIP_INVALID_ARGUMENT, "pooled feature with occurrences but no bags");
    if (f.pooling == EPS_HIP_POOL_WEIGHTED_SUM && f.occurrences && !f.weights)
      return Fail(EPS_HIP_INVALID_ARGUMENT, "weighted feature needs weights");
    const uint64_t rows = f.pooling == EPS_HIP_POOL_SEQUENCE ? f.occurrences : f.bags;
    if (rows >= (1ull << kRefRowBits)) return Fail(EPS_HIP_CAPACITY_EXCEEDED, "feature has too many rows");
    plan.occurrences += f.occurrences;
    plan.class_occurrences[DimClass(tables[f.table].dim)] += f.occurrences;
  }
  if (plan.occurrences >= (1ull << 30)) return Fail(EPS_HIP_CAPACITY_EXCEEDED, "too many occurrences");
  return EPS_HIP_OK;
}

// Final sorted buffers after `passes` passes starting from A.
inline bool SortedInB(uint32_t passes) { return passes % 2 == 1; }

}  // namespace eps_hip

using namespace eps_hip;

extern "C" {

uint64_t eps_hip_push_workspace_bytes(uint64_t occurrences) {
  return PushLayout(occurrences).total;
}

}  // extern "C"

namespace eps_hip {
namespace {
int Prepare(const eps_hip_table* tables, uint32_t table_count, const eps_hip_push_feature* features,
            uint32_t feature_count, void* workspace, uint64_t workspace_bytes, void* stream, bool with_vals) {
  PushPlan plan;
  EPS_HIP_TRY(PlanPush(tables, table_count, features, feature_count, plan));
  const PushLayout L(plan.occurrences);
  if (!workspace || workspace_bytes < L.total)
    return Fail(EPS_HIP_CAPACITY_EXCEEDED, "push workspace too small");
  auto* ws = static_cast<uint8_t*>(workspace);
  auto* ctrl = reinterpret_cast<Control*>(ws);
  const hipStream_t s = AsStream(stream);
  // Control block (but its status history), histograms and the look-back
  // flags of the passes this push sorts with start at zero (the group
  // look-back flags are cleared by keygen, below).
  if (!plan.occurrences)
    return LaunchFill(reinterpret_cast<uint32_t*>(ws), 0, sizeof(Control) / 4, s, kHistoryWord);
  EPS_HIP_TRY(LaunchFill(reinterpret_cast<uint32_t*>(ws), 0, (L.look + plan.passes * L.tiles * kDigits * 4) / 4, s,
                         kHistoryWord));

  PrepArgs args{};
  args.count = feature_count;
  args.row_bits = plan.row_bits;
  args.sentinel = plan.key_bits >= 32 ? 0xffffffffu : ((1u << plan.key_bits) - 1);
  args.passes = plan.passes;
  for (uint32_t p = 0; p < kMaxPasses; ++p) { args.shift[p] = plan.shift[p]; args.bits[p] = plan.bits[p]; }
  args.ctrl = ctrl;
  args.hist = reinterpret_cast<uint32_t*>(ws + L.hist);
  args.keys = reinterpret_cast<uint32_t*>(ws + L.keys_a);
  args.vals = with_vals ? reinterpret_cast<uint32_t*>(ws + L.vals_a) : nullptr;
  args.zero = reinterpret_cast<uint32_t*>(ws + L.group_look);
  args.zero_words = uint64_t(plan.passes) * L.groups * kDigits;
  // Reference words ping-pong between two buffers through the passes and
  // end in sorted_rs: keygen writes them where an even number of swaps
  // before the end starts.  A push with no weighted-sum feature sorts them
  // as 4-byte words without their scales (a third less sort traffic) and the
  // last pass puts the scales back.
  uint64_t* rs[2] = {reinterpret_cast<uint64_t*>(ws + (plan.passes % 2 ? L.refscale : L.sorted_rs)),
                     reinterpret_cast<uint64_t*>(ws + (plan.passes % 2 ? L.sorted_rs : L.refscale))};
  ScaleArgs sc{};
  bool narrow = true;
  for (uint32_t i = 0; i < feature_count; ++i) {
    if (features[i].pooling == EPS_HIP_POOL_WEIGHTED_SUM) narrow = false;
    if (features[i].pooling == EPS_HIP_POOL_MEAN) {
      sc.mean_mask |= 1u << i;
      sc.lengths[i] = features[i].valid_lengths;
    }
  }
  args.refscale = narrow ? nullptr : rs[0];
  args.refs = narrow ? reinterpret_cast<uint32_t*>(rs[0]) : nullptr;
  uint64_t occ = 0, blocks = 0;
  for (uint32_t i = 0; i < feature_count; ++i) {
    const auto& in = features[i];
    PrepFeature& f = args.f[i];
    f.indices = in.indices; f.offsets = in.offsets; f.lengths = in.valid_lengths;
    f.weights = in.weights; f.occ_begin = occ; f.occurrences = in.occurrences; f.bags = in.bags;
    f.table_rows = tables[in.table].rows; f.key_index = plan.key_index[in.table];
    f.pooling = in.pooling; f.feature = i; f.block_begin = uint32_t(blocks);
    occ += in.occurrences;
    blocks += (in.occurrences + kBlock * kKeygenItems - 1) / (kBlock * kKeygenItems);
  }
  if (blocks) {
    hipLaunchKernelGGL(KeygenKernel, dim3(unsigned(blocks)), dim3(kBlock), 0, s, args);
    EPS_HIP_LAUNCHED("keygen");
  }
  uint32_t* keys[2] = {reinterpret_cast<uint32_t*>(ws + L.keys_a), reinterpret_cast<uint32_t*>(ws + L.keys_b)};
  uint32_t* vals[2] = {reinterpret_cast<uint32_t*>(ws + L.vals_a), reinterpret_cast<uint32_t*>(ws + L.vals_b)};
  auto* look = reinterpret_cast<uint32_t*>(ws + L.look);
  auto* group_look = reinterpret_cast<uint32_t*>(ws + L.group_look);
  const uint32_t n = uint32_t(plan.occurrences);
  for (uint32_t p = 0; p < plan.passes; ++p) {
    const int form = !narrow ? kWide : (p + 1 < plan.passes ? kNarrow : kWiden);
    auto launch = [&](auto kernel, const auto* in, auto* out) {
      hipLaunchKernelGGL(kernel, dim3(unsigned(L.tiles)), dim3(kBlock), 0, s, keys[p % 2], vals[p % 2],
                         keys[(p + 1) % 2], vals[(p + 1) % 2], in, out, n, plan.shift[p], plan.bits[p],
                         args.hist + p * kDigits, look + uint64_t(p) * L.tiles * kDigits,
                         group_look + uint64_t(p) * L.groups * kDigits, uint32_t(L.tiles), &ctrl->tile_counter[p],
                         sc);
    };
    const uint64_t* in8 = rs[p % 2];
    uint64_t* out8 = rs[(p + 1) % 2];
    const uint32_t* in4 = reinterpret_cast<const uint32_t*>(rs[p % 2]);
    uint32_t* out4 = reinterpret_cast<uint32_t*>(rs[(p + 1) % 2]);
    if (form == kWide)
      launch(with_vals ? RadixPassKernel<true, kWide> : RadixPassKernel<false, kWide>, in8, out8);
    else if (form == kNarrow)
      launch(with_vals ? RadixPassKernel<true, kNarrow> : RadixPassKernel<false, kNarrow>, in4, out4);
    else
      launch(with_vals ? RadixPassKernel<true, kWiden> : RadixPassKernel<false, kWiden>, in4, out8);
    EPS_HIP_LAUNCHED("radix pass");
  }
  // Hot rows of the sorted keys.
  HotArgs ha{};
  ha.keys = keys[plan.passes % 2];
  ha.hot = reinterpret_cast<HotEntry*>(ws + L.long_list);
  ha.ctrl = ctrl;
  ha.n = n;
  ha.row_bits = plan.row_bits;
  ha.capacity = uint32_t(L.HotCapacity());
  ha.sentinel = args.sentinel;
  for (uint32_t c = 0; c <= kClasses; ++c) ha.class_key[c] = plan.class_start[c];
  ha.class_key[kClasses] = table_count;
  hipLaunchKernelGGL(HotListKernel, dim3(unsigned(n / kBlock + 1)), dim3(kBlock), 0, s, ha);
  EPS_HIP_LAUNCHED("hot rows");
  return EPS_HIP_OK;
}
}  // namespace

int PrepareWithOccurrences(const eps_hip_table* tables, uint32_t table_count,
                           const eps_hip_push_feature* features, uint32_t feature_count, void* workspace,
                           uint64_t workspace_bytes, void* stream) {
  return Prepare(tables, table_count, features, feature_count, workspace, workspace_bytes, stream, true);
}
}  // namespace eps_hip

extern "C" {

int eps_hip_prepare(const eps_hip_table* tables, uint32_t table_count,
                    const eps_hip_push_feature* features, uint32_t feature_count,
                    void* workspace, uint64_t workspace_bytes, void* stream) {
  return Prepare(tables, table_count, features, feature_count, workspace, workspace_bytes, stream, false);
}

int eps_hip_unique(const eps_hip_table* tables, uint32_t table_count,
                   const eps_hip_push_feature* features, uint32_t feature_count,
                   void* workspace, uint64_t workspace_bytes, uint64_t* unique_slots,
                   uint32_t* unique_tables, uint64_t* occurrence_to_unique,
                   uint64_t* unique_count, void* stream) {
  PushPlan plan;
  EPS_HIP_TRY(PlanPush(tables, table_count, features, feature_count, plan));
  const PushLayout L(plan.occurrences);
  if (!workspace || workspace_bytes < L.total)
    return Fail(EPS_HIP_CAPACITY_EXCEEDED, "push workspace too small");
  if (!unique_slots || !unique_tables || !occurrence_to_unique)
    return Fail(EPS_HIP_INVALID_ARGUMENT, "null unique outputs");
  EPS_HIP_TRY(PrepareWithOccurrences(tables, table_count, features, feature_count, workspace, workspace_bytes,
                                     stream));
  auto* ws = static_cast<uint8_t*>(workspace);
  auto* ctrl = reinterpret_cast<Control*>(ws);
  const hipStream_t s = AsStream(stream);
  const uint32_t n = uint32_t(plan.occurrences);
  // Holes keep UINT64_MAX (include/eps/types.hpp:139; cache_backend.cu:281).
  EPS_HIP_TRY(LaunchFill(reinterpret_cast<uint32_t*>(occurrence_to_unique), 0xffffffffu, 2ull * n, s));
  if (!n) {
    if (unique_count) EPS_HIP_TRY(LaunchFill(reinterpret_cast<uint32_t*>(unique_count), 0, 2, s));
    return EPS_HIP_OK;
  }
  const bool in_b = SortedInB(plan.passes);
  const auto* keys = reinterpret_cast<const uint32_t*>(ws + (in_b ? L.keys_b : L.keys_a));
  const auto* vals = reinterpret_cast<const uint32_t*>(ws + (in_b ? L.vals_b : L.vals_a));
  auto* flags = reinterpret_cast<uint32_t*>(ws + L.flags);
  auto* ranks = reinterpret_cast<uint32_t*>(ws + L.ranks);
  auto* sums = reinterpret_cast<uint32_t*>(ws + L.block_sums);
  const uint32_t scan_blocks = (n + 1023) / 1024;
  EPS_HIP_TRY(LaunchFill(flags, 0, n, s));
  if (unique_count) EPS_HIP_TRY(LaunchFill(reinterpret_cast<uint32_t*>(unique_count), 0, 2, s));
  hipLaunchKernelGGL(HeadFlagKernel, dim3(Grid(n, 8192)), dim3(kBlock), 0, s, keys, vals, ctrl, flags, n);
  EPS_HIP_LAUNCHED("head flags");
  hipLaunchKernelGGL(ScanBlockSumsKernel, dim3(scan_blocks), dim3(kBlock), 0, s, flags, sums, n);
  EPS_HIP_LAUNCHED("scan sums");
  hipLaunchKernelGGL(ScanTopKernel, dim3(1), dim3(kBlock), 0, s, sums, scan_blocks, ctrl, unique_count);
  EPS_HIP_LAUNCHED("scan top");
  hipLaunchKernelGGL(ScanApplyKernel, dim3(scan_blocks), dim3(kBlock), 0, s, flags, sums, ranks, n);
  EPS_HIP_LAUNCHED("scan apply");
  UniqueArgs uargs{};
  for (uint32_t k = 0; k < table_count; ++k) uargs.table_of_key[k] = plan.table_of_key[k];
  hipLaunchKernelGGL(UniqueWriteKernel, dim3(Grid(n, 8192)), dim3(kBlock), 0, s, keys, vals, ranks,
                     ctrl, n, plan.row_bits, uargs, unique_slots, unique_tables,
                     occurrence_to_unique);
  EPS_HIP_LAUNCHED("unique write");
  return EPS_HIP_OK;
}

}  // extern "C"
