// adam.hip -- duplicate-id aggregation fused with sparse (Lazy)Adam.
//
// Per unique row, one sub-wavefront group of G lanes (lane l owns columns
// [4l, 4l+4)) sums the row's references in order from +0.0f -- acc = acc +
// src * scale, separate multiply and add -- (ReduceGradients,
// src/access/batch_access.cpp:73-93; ExpandCompactGradients,
// src/access/compact_gradients.cpp:31-36; ReduceFeatureGradients,
// src/cuda/cache_backend.cu:115-125), then reads the row's w, m, v once, applies
//   m' = b1*m + (1-b1)*g;  v' = b2*v + ((1-b2)*g)*g;  w' = w - (lr_t*m')/(sqrt(v')+eps)
// and the clamp (src/update/lazy_adam.cpp:31-35; AdamKernel,
// src/cuda/cache_backend.cu:95-114), and writes w, m, v once.
//
// All-or-nothing without a second pass over the state.  The reference
// validates every element before any write, with a second full state pass
// (ValidateLazyAdam then ApplyLazyAdam; AdamKernel twice).  Here a guard decides
// before the update whether overflow is impossible:
//   * bounds domain: running maxima W >= |w|, M >= |m|, V >= v of every value
//     this library ever wrote (init, admission, updates);
//   * G >= |g| for every reduced gradient: max|source| * max(1, max|scale|) *
//     references * (1+2^-24)^(references+2) (rounding growth of a sequential sum);
//   * then |m'| <= b1*M + (1-b1)*G, v' <= b2*V + (1-b2)*G^2 and
//     |w'| <= W + lr_t*|m'|/eps (since sqrt(v') + eps >= eps), each widened by 1%.
// If every bound stays below 1e30 (far below FLT_MAX) no element can overflow and
// the single fused pass runs ("fused").  Otherwise the same kernel runs in
// validate-only mode and a second launch applies only if nothing failed
// ("checked") -- the reference's two-pass behaviour.  A non-finite gradient value
// or an out-of-range slot rejects the whole update before anything is written.
#include "prepare.hpp"

#include <hip/hip_ext.h>

#include <algorithm>
#include <atomic>
#include <cfloat>
#include <cmath>

namespace eps_hip {

namespace {

constexpr uint32_t kFallbackGrid = 2048;

// ---------------------------------------------------------------------------
// Gradient scan (GradMaxKernel), the first kernel of an update.  Its spans are
// the guarded input arrays: gradient values, reference scales, 64-bit caller
// indices that must all be below `limit`, and (a push) the sorted keys of the
// prepared workspace, whose table indices and slots must name the push's
// tables and rows.  It records max |gradient| and max |scale| for the guard
// and any range failure as a prepare-time finding, all before anything is
// written; block 0 also copies the bounds-domain maxima into the control
// block, the snapshot the guard decides from.  (The reference words are
// checked where the update kernels decode them: a word naming no gradient row
// of the push is never used as an address, and the rows it feeds are not
// written.)
enum SpanKind : uint32_t { kGradientSpan = 0, kScaleSpan = 1, kIndexSpan = 2, kSortedSpan = 3 };
struct Span {
  const float* p;
  uint64_t count;
  uint32_t block_begin, kind;
  uint64_t limit;
};
// What the sorted keys are checked against (key index order for tables).
struct SortedCheck {
  const uint32_t* keys;
  uint64_t table_rows[EPS_HIP_MAX_TABLES];
  uint32_t row_bits, tables;
};
struct GuardArgs {
  Span span[EPS_HIP_MAX_FEATURES + 4];
  uint32_t spans;
  Control* ctrl;
  const Bounds* bounds;  // snapshot source (NULL: no snapshot)
  SortedCheck sorted;
};
static_assert(sizeof(GuardArgs) <= 4096, "gradient scan arguments fit the kernel-argument segment");
constexpr uint32_t kMaxItems = 16;     // float4 per thread per block (all issued before any is used)
constexpr uint32_t kSortedItems = 16;  // sorted keys per thread per block

__global__ void __launch_bounds__(kBlock) GradMaxKernel(GuardArgs a) {
  __shared__ uint32_t s_max[4];
  __shared__ uint64_t s_rows[EPS_HIP_MAX_TABLES];
  if (blockIdx.x == 0 && threadIdx.x < kWave && a.bounds) {
    const uint32_t lane = threadIdx.x;
    const uint32_t w = WaveMax(a.bounds->v[lane][0]), m = WaveMax(a.bounds->v[lane][1]),
                   v = WaveMax(a.bounds->v[lane][2]);
    if (lane == 0) {
      a.ctrl->snap[0] = w;
      a.ctrl->snap[1] = m;
      a.ctrl->snap[2] = v;
    }
  }
  if (!a.spans) return;
  const Span sp = a.span[PartOf(a.span, a.spans)];
  uint32_t m = 0;
  uint32_t found = 0;  // prepare-status bits this thread found
  if (sp.kind == kSortedSpan) {
    const SortedCheck& c = a.sorted;
    if (threadIdx.x < EPS_HIP_MAX_TABLES) s_rows[threadIdx.x] = c.table_rows[threadIdx.x];
    __syncthreads();
    // Positions past the valid count hold keys of rows not on this device,
    // which no update kernel reads.
    const uint64_t per_block = uint64_t(kBlock) * kSortedItems;
    const uint64_t begin = uint64_t(blockIdx.x - sp.block_begin) * per_block;
    {
      // Every load is issued before any is used (and before the valid count
      // is known): positions past the span read the block's first position,
      // and positions past the valid count are not judged.
      uint32_t key[kSortedItems];
#pragma unroll
      for (uint32_t k = 0; k < kSortedItems; ++k) {
        const uint64_t i = begin + uint64_t(k) * kBlock + threadIdx.x;
        key[k] = c.keys[i < sp.count ? i : begin];
      }
      const uint64_t valid = min<uint64_t>(sp.count, a.ctrl->valid_count);
      bool bad = false;
#pragma unroll
      for (uint32_t k = 0; k < kSortedItems; ++k) {
        const uint64_t i = begin + uint64_t(k) * kBlock + threadIdx.x;
        const KeyParts kp = SplitKey(key[k], c.row_bits);
        bad |= i < valid && !KeyInRange(kp, c.tables, s_rows[min(kp.table, EPS_HIP_MAX_TABLES - 1u)]);
      }
      if (bad) found = EPS_HIP_STATUS_BAD_INDEX;
    }
  } else if (sp.kind == kIndexSpan) {
    const uint64_t per_block = uint64_t(kBlock) * kMaxItems * 4;
    const uint64_t begin = uint64_t(blockIdx.x - sp.block_begin) * per_block;
    const uint64_t end = min(begin + per_block, sp.count);
    const uint64_t* idx = reinterpret_cast<const uint64_t*>(sp.p);
    for (uint64_t i = begin + threadIdx.x; i < end; i += kBlock)
      if (idx[i] >= sp.limit) found = EPS_HIP_STATUS_BAD_INDEX;
  } else {
    const uint64_t per_block = uint64_t(kBlock) * kMaxItems * 4;
    const uint64_t begin = uint64_t(blockIdx.x - sp.block_begin) * per_block;
    const uint64_t end = min(begin + per_block, sp.count);
    if (reinterpret_cast<uintptr_t>(sp.p) % 16 == 0) {
      const uint64_t vend = begin + ((end - begin) & ~uint64_t(3));
      // Every load is issued before any is used (a branch around each would
      // make the compiler wait for each pair): quads past the vector part
      // read the block's first quad and count as zeros.
      float4 x[kMaxItems];
      if (vend > begin) {  // uniform over the block
#pragma unroll
        for (uint32_t k = 0; k < kMaxItems; ++k) {
          const uint64_t i = begin + (uint64_t(k) * kBlock + threadIdx.x) * 4;
          x[k] = Load4(sp.p + (i < vend ? i : begin));
        }
#pragma unroll
        for (uint32_t k = 0; k < kMaxItems; ++k) {
          const uint64_t i = begin + (uint64_t(k) * kBlock + threadIdx.x) * 4;
          if (i >= vend) x[k] = make_float4(0.f, 0.f, 0.f, 0.f);
        }
      } else {
#pragma unroll
        for (uint32_t k = 0; k < kMaxItems; ++k) x[k] = make_float4(0.f, 0.f, 0.f, 0.f);
      }
      uint32_t neg = 0;  // any value below zero (not -0.0)
#pragma unroll
      for (uint32_t k = 0; k < kMaxItems; ++k) {
        m = max(m, max(max(AbsBits(x[k].x), AbsBits(x[k].y)), max(AbsBits(x[k].z), AbsBits(x[k].w))));
        neg |= (x[k].x < 0.f) | (x[k].y < 0.f) | (x[k].z < 0.f) | (x[k].w < 0.f);
      }
      for (uint64_t i = vend + threadIdx.x; i < end; i += kBlock) {
        m = max(m, AbsBits(sp.p[i]));
        neg |= sp.p[i] < 0.f;
      }
      if (sp.kind == kScaleSpan && neg) found = EPS_HIP_STATUS_BAD_SCALE;
    } else {
      for (uint64_t i = begin + threadIdx.x; i < end; i += kBlock) {
        m = max(m, AbsBits(sp.p[i]));
        if (sp.kind == kScaleSpan && sp.p[i] < 0.f) found = EPS_HIP_STATUS_BAD_SCALE;
      }
    }
    // A compact scale must be finite and >= 0 (compact_gradients.cpp:21).
    if (sp.kind == kScaleSpan && m >= 0x7f800000u) found = EPS_HIP_STATUS_BAD_SCALE;
  }
  if (found) atomicOr(&a.ctrl->prep_status, found);
  m = WaveMax(m);
  if ((threadIdx.x & (kWave - 1)) == 0) s_max[threadIdx.x / kWave] = m;
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t bm = max(max(s_max[0], s_max[1]), max(s_max[2], s_max[3]));
    if (bm)
      atomicMax(sp.kind == kScaleSpan ? &a.ctrl->scale_slots[blockIdx.x % kSrcSlots]
                                      : &a.ctrl->src_slots[blockIdx.x % kSrcSlots], bm);
  }
}

// ---------------------------------------------------------------------------
// Shared per-row arithmetic.
struct TableDesc {
  float* state;
  uint64_t rows;     // slots of the table (sorted keys must name one)
  uint32_t dim;
  float beta1, beta2, omb1, omb2, lr, eps, lo, hi;
  uint32_t bounded;  // lo/hi are the table's weight bounds (else -FLT_MAX/FLT_MAX)
};

// Running maxima of magnitude bits over a thread's elements: of the reduced
// gradients (bg), and of m, v and w (before and after the clamp) as computed.
// A maximum at or above the infinity pattern means a non-finite value; the
// m, v, w maxima of what a launch writes feed the bounds domain.
struct RowStats {
  uint32_t err = 0, bg = 0, bw = 0, bm = 0, bv = 0;
};

// Block-wide copy of a kernel-argument array to LDS, one 32-bit word per
// thread per step (the arrays are read in place from the argument segment).
template <uint32_t kThreads = kBlock>
__device__ __forceinline__ void CopyWords(void* dst, const void* src, uint32_t bytes) {
  const uint32_t* from = static_cast<const uint32_t*>(src);
  uint32_t* to = static_cast<uint32_t*>(dst);
  for (uint32_t i = threadIdx.x; i < bytes / 4; i += kThreads) to[i] = from[i];
}

// Correctly rounded square root.  For x in [2^-96, infinity) it is the
// hardware estimate s corrected to s - 1 ulp or s + 1 ulp by the signs of the
// residuals fma(-(s -/+ ulp), s, x): the steps hipcc emits for sqrtf once its
// range handling (scaling of tiny inputs, zero and infinity) is out of the
// way, so both give the same bits.  Other inputs take sqrtf.
__device__ __forceinline__ float SqrtRn(float x) {
  const uint32_t b = __float_as_uint(x);
  if (b - 0x0f800000u < 0x7f800000u - 0x0f800000u) {
    const float s = __builtin_amdgcn_sqrtf(x);
    const float below = __uint_as_float(__float_as_uint(s) - 1u);
    const float above = __uint_as_float(__float_as_uint(s) + 1u);
    const float r = fmaf(-below, s, x) <= 0.f ? below : s;
    return fmaf(-above, s, x) > 0.f ? above : r;
  }
  return sqrtf(x);
}

// One element: Adam in the reference's operation order, w clamped to the
// table's bounds (kClamp false: an unbounded table, whose clamp to
// -FLT_MAX..FLT_MAX changes no finite w, and a non-finite w is an error that
// nothing is written for).  vn is +0 or more, or NaN (v >= 0 and
// (omb2 * g) * g >= 0), so its raw bits order like its magnitude.
template <bool kClamp = true>
__device__ __forceinline__ void AdamElement(const TableDesc& T, float g, float& w, float& m,
                                            float& v, RowStats& st) {
  const float mn = T.beta1 * m + T.omb1 * g;
  const float vn = T.beta2 * v + (T.omb2 * g) * g;
  const float wn = w - (T.lr * mn) / (SqrtRn(vn) + T.eps);
  st.bg = max(st.bg, AbsBits(g));
  st.bm = max(st.bm, AbsBits(mn));
  st.bv = max(st.bv, __float_as_uint(vn));
  if (kClamp) {
    w = Clamp(wn, T.lo, T.hi);
    st.bw = max(st.bw, max(AbsBits(wn), AbsBits(w)));
  } else {
    w = wn;
    st.bw = max(st.bw, AbsBits(wn));
  }
  m = mn;
  v = vn;
}

// Vector row update: lane owns columns [c, c+4).
__device__ __forceinline__ void AdamRow4(const TableDesc& T, uint64_t slot, uint32_t c, float4 g,
                                         bool write, RowStats& st) {
  float* row = T.state + slot * uint64_t(T.dim) * 3;
  float4 w = Load4(row + c), m = Load4(row + T.dim + c), v = Load4(row + 2 * T.dim + c);
  AdamElement(T, g.x, w.x, m.x, v.x, st);
  AdamElement(T, g.y, w.y, m.y, v.y, st);
  AdamElement(T, g.z, w.z, m.z, v.z, st);
  AdamElement(T, g.w, w.w, m.w, v.w, st);
  if (write) {
    Store4(row + c, w);
    Store4(row + T.dim + c, m);
    Store4(row + 2 * T.dim + c, v);
  }
}

__device__ __forceinline__ void AdamRow1(const TableDesc& T, uint64_t slot, uint32_t c, float g,
                                         bool write, RowStats& st) {
  float* row = T.state + slot * uint64_t(T.dim) * 3;
  float w = LoadF(row + c), m = LoadF(row + T.dim + c), v = LoadF(row + 2 * T.dim + c);
  AdamElement(T, g, w, m, v, st);
  if (write) {
    StoreF(row + c, w); StoreF(row + T.dim + c, m); StoreF(row + 2 * T.dim + c, v);
  }
}

__device__ __forceinline__ void Accumulate4(float4& acc, float4 x, float s) {
  acc.x = acc.x + x.x * s;
  acc.y = acc.y + x.y * s;
  acc.z = acc.z + x.z * s;
  acc.w = acc.w + x.w * s;
}

// The guard decision (see the file comment), made by every block of the first
// kernel of an update from inputs that earlier kernels wrote and nothing
// changes while the update runs: the gradient maxima, the prepare-time
// findings and the bounds snapshot the gradient scan took (never the live
// bounds domain, which the update's own finished blocks raise).  So every
// block -- of either kernel, when two decide on two streams -- takes the same
// decision.  Block 0 publishes the mode and the status bits for the kernels
// after it.  Runs in wavefront 0 (one gradient slot and one table per lane);
// returns the mode to every thread.
static_assert(kSrcSlots == kWave, "one guard slot per lane");
struct GuardScalars {
  uint64_t refs;       // references summed into one reduced gradient, at most; 0: the prepared count
  uint32_t tables;
};
__device__ uint32_t DecideBlock(Control* ctrl, const TableDesc* t, const GuardScalars& gs, uint32_t* s_mode) {
  if (threadIdx.x < kWave) {
    const uint32_t lane = threadIdx.x;
    const uint32_t gb = WaveMax(ctrl->src_slots[lane]);
    const uint32_t scale_bits = WaveMax(ctrl->scale_slots[lane]);
    uint32_t status = ctrl->prep_status;
    uint32_t mode = kFused;
    if (status & (EPS_HIP_STATUS_BAD_INDEX | EPS_HIP_STATUS_BAD_SCALE)) {
      mode = kReject;
    } else if (gb >= 0x7f800000u) {
      status |= EPS_HIP_STATUS_NONFINITE_GRAD;
      mode = kReject;
    } else if (scale_bits >= 0x7f800000u) {  // a non-finite weight or scale
      status |= EPS_HIP_STATUS_BAD_SCALE;
      mode = kReject;
    } else {
      const double W = __uint_as_float(ctrl->snap[0]), M = __uint_as_float(ctrl->snap[1]),
                   V = __uint_as_float(ctrl->snap[2]);
      const double refs = double(gs.refs ? gs.refs : uint64_t(ctrl->valid_count));
      const double G = GuardGradBound(__uint_as_float(gb), __uint_as_float(scale_bits), refs);
      bool table_safe = true;  // one table per lane
      if (lane < gs.tables) {
        const TableDesc& T = t[lane];
        table_safe = GuardTableSafe(T.beta1, T.beta2, T.lr, T.eps, W, M, V, G);
      }
      if (!(G < kGuardLimit) || __ballot(!table_safe) != 0) {
        mode = kChecked;
        status |= EPS_HIP_STATUS_CHECKED_PATH;
      }
    }
    if (mode == kReject) status |= EPS_HIP_STATUS_REJECTED;
    if (lane == 0) {
      *s_mode = mode;
      if (blockIdx.x == 0) {
        ctrl->mode = mode;
        ReportStatus(ctrl, status);
      }
    }
  }
  __syncthreads();
  return *s_mode;
}

// Role of a launch in an update.  The first kernel decides (DecideBlock);
// the primary kernels after it follow that decision; the fallback (the apply
// pass of the checked path) runs only when the decision was "checked" and the
// validate-only pass found nothing.
enum Role : uint32_t { kDecide = 0, kFollow = 1, kFallback = 2 };

// Whether this launch has work, and whether it writes (uniform over the
// block).  s_t must hold the launch's tables; every thread calls it.
__device__ bool LaunchGate(Control* ctrl, const TableDesc* s_t, const GuardScalars& gs, uint32_t role,
                           uint32_t* s_mode, bool& write) {
  if (role == kDecide) {
    __syncthreads();  // s_t is staged
    const uint32_t mode = DecideBlock(ctrl, s_t, gs, s_mode);
    write = mode == kFused;
    return mode != kReject;
  }
  const uint32_t mode = ctrl->mode, status = ctrl->status;
  if (role == kFollow) {
    // A stall in an earlier kernel of a fused update stops every later write.
    write = mode == kFused;
    return mode != kReject && !(status & EPS_HIP_STATUS_STALLED);
  }
  if (mode != kChecked) return false;
  if (status & (kErrorBits | EPS_HIP_STATUS_STALLED)) {
    if (blockIdx.x == 0 && threadIdx.x == 0) ReportStatus(ctrl, EPS_HIP_STATUS_REJECTED);
    return false;
  }
  write = true;
  return true;
}

// Block-level fold of the per-lane statistics: error bits (with those the
// maxima imply) to the status word, written maxima to one slot of the bounds
// domain.
template <uint32_t kWaves = kBlock / kWave>
__device__ void FinishBlock(const RowStats& st, Control* ctrl, Bounds* bounds, bool wrote) {
  __shared__ uint32_t s_red[kWaves][4];
  uint32_t e = st.err;
  if (st.bg >= 0x7f800000u) e |= EPS_HIP_STATUS_REDUCE_OVERFLOW;
  if (max(st.bw, max(st.bm, st.bv)) >= 0x7f800000u) e |= EPS_HIP_STATUS_ADAM_OVERFLOW;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) e |= uint32_t(__shfl_xor(int(e), o));
  const uint32_t w = WaveMax(st.bw), m = WaveMax(st.bm), v = WaveMax(st.bv);
  const uint32_t wave = threadIdx.x / kWave;
  if ((threadIdx.x & (kWave - 1)) == 0) {
    s_red[wave][0] = e; s_red[wave][1] = w; s_red[wave][2] = m; s_red[wave][3] = v;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t E = 0, W = 0, M = 0, V = 0;
    for (uint32_t i = 0; i < kWaves; ++i) {
      E |= s_red[i][0]; W = max(W, s_red[i][1]); M = max(M, s_red[i][2]); V = max(V, s_red[i][3]);
    }
    ReportStatus(ctrl, E);
    if (wrote && bounds) {
      uint32_t* slot = bounds->v[blockIdx.x % kBoundSlots];
      if (W) atomicMax(slot + 0, W);
      if (M) atomicMax(slot + 1, M);
      if (V) atomicMax(slot + 2, V);
    }
  }
}

// ---------------------------------------------------------------------------
// Sorted driver: segments are runs of equal keys in the sorted key array.
struct FusedArgs {
  TableDesc t[EPS_HIP_MAX_TABLES];   // by key index
  const float* grad[EPS_HIP_MAX_FEATURES];
  uint64_t grad_rows[EPS_HIP_MAX_FEATURES];
  const uint32_t* keys;
  const uint64_t* rs;
  const uint32_t* vals;              // reduce mode: sorted occurrence indices
  const uint64_t* occ2u;             // reduce mode
  float* reduce_out;
  uint64_t reduce_stride;
  Control* ctrl;
  Bounds* bounds;
  GuardScalars gs;
  uint32_t row_bits, cls, cls_end, log2g, ppb, vblocks, role, reduce, tables, features;  // classes [cls, cls_end)
  uint32_t n;  // occurrences of the push (sorted positions, occurrence indices)
};
static_assert(sizeof(FusedArgs) <= 4096, "update arguments fit the kernel-argument segment");

template <bool kGeneric>
__global__ void __launch_bounds__(kBlock) SortedUpdateKernel(FusedArgs a) {
  __shared__ TableDesc s_t[EPS_HIP_MAX_TABLES];
  __shared__ const float* s_grad[EPS_HIP_MAX_FEATURES];
  __shared__ uint32_t s_heads[kBlock];
  __shared__ uint32_t s_wave_heads[4];
  __shared__ uint32_t s_mode;
  __shared__ uint64_t s_rows[EPS_HIP_MAX_FEATURES];  // gradient rows per feature
  CopyWords(s_t, a.t, sizeof(a.t));
  CopyWords(s_grad, a.grad, sizeof(a.grad));
  CopyWords(s_rows, a.grad_rows, sizeof(a.grad_rows));
  Control* ctrl = a.ctrl;
  bool write = true;
  if (!a.reduce && !LaunchGate(ctrl, s_t, a.gs, a.role, &s_mode, write)) return;
  // The classes' sorted positions, from the workspace, kept inside the push's.
  const uint32_t first = ctrl->class_start[a.cls], last = ctrl->class_start[a.cls_end];
  const uint32_t end = min(last, a.n), start = min(first, end);
  const uint32_t G = kGeneric ? kWave : (1u << a.log2g);
  const uint32_t lig = threadIdx.x & (G - 1);
  const uint32_t gid = threadIdx.x / G, ngroups = kBlock / G;
  const uint32_t lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  RowStats st;
  __syncthreads();
  for (uint32_t vb = blockIdx.x; vb < a.vblocks; vb += gridDim.x) {
    const uint32_t p0 = start + vb * a.ppb;
    if (p0 >= end) break;  // uniform: later virtual blocks are further right
    const uint32_t p1 = min(p0 + a.ppb, end);
    // Head positions of this block's range, in order.
    const uint32_t p = p0 + threadIdx.x;
    const bool head = threadIdx.x < a.ppb && p < p1 && (p == start || a.keys[p] != a.keys[p - 1]);
    const uint64_t ballot = __ballot(head);
    if (lane == 0) s_wave_heads[wave] = uint32_t(__popcll(ballot));
    __syncthreads();
    uint32_t before = 0;
    for (uint32_t w = 0; w < wave; ++w) before += s_wave_heads[w];
    const uint32_t nheads = s_wave_heads[0] + s_wave_heads[1] + s_wave_heads[2] + s_wave_heads[3];
    if (head) s_heads[before + uint32_t(__popcll(ballot & ((1ull << lane) - 1)))] = p;
    __syncthreads();
    for (uint32_t h = gid; h < nheads; h += ngroups) {
      const uint32_t sb = s_heads[h];
      const uint32_t key = a.keys[sb];
      const uint32_t se = h + 1 < nheads ? s_heads[h + 1] : SegmentEndSearch(a.keys, p1, end, key);
      // A key or reference naming nothing of the push (a damaged workspace)
      // is not used as an address: its loads read zero and the row is not
      // written.  The reference checks see the same words in every lane.
      const KeyParts kp = SplitKey(key, a.row_bits);
      const TableDesc& T = s_t[min(kp.table, a.tables - 1)];
      bool ok = KeyInRange(kp, a.tables, T.rows) && (!a.reduce || a.vals[sb] < a.n);
      const uint64_t slot = ok ? kp.slot : 0;
      const uint32_t dim = T.dim;
      const uint64_t u = a.reduce && ok ? a.occ2u[a.vals[sb]] : 0;
      auto ref_ok = [&](uint64_t w) {
        const RefParts rp = SplitRef(w);
        return RefInRange(rp, a.features, s_rows[min(rp.feature, a.features - 1)]);
      };
      if (!kGeneric) {
        const uint32_t c = lig * 4;
        const bool active = c < dim;
        float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
        for (uint32_t base = sb; base < se; base += G) {
          const uint32_t cnt = min(G, se - base);
          const uint64_t my = lig < cnt ? a.rs[base + lig] : 0ull;
          for (uint32_t k = 0; k < cnt; k += 4) {
            float4 x[4];
            float s[4];
#pragma unroll
            for (uint32_t q = 0; q < 4; ++q) {
              const uint64_t w = __shfl(my, int(k + q), int(G));
              const uint32_t ref = uint32_t(w);
              s[q] = __uint_as_float(uint32_t(w >> 32));
              const bool in = k + q < cnt && ref_ok(w);
              if (k + q < cnt && !in) ok = false;
              const float* src = s_grad[ref >> kRefRowBits] +
                                 uint64_t(ref & ((1u << kRefRowBits) - 1)) * dim + c;
              x[q] = (in && active) ? Load4(src) : make_float4(0.f, 0.f, 0.f, 0.f);
            }
#pragma unroll
            for (uint32_t q = 0; q < 4; ++q)
              if (k + q < cnt) Accumulate4(acc, x[q], s[q]);
          }
        }
        if (!ok) st.err |= EPS_HIP_STATUS_BAD_INDEX;
        if (!active || !ok) continue;
        if (a.reduce) {
          if (!(Finite(acc.x) && Finite(acc.y) && Finite(acc.z) && Finite(acc.w)))
            st.err |= EPS_HIP_STATUS_REDUCE_OVERFLOW;
          Store4(a.reduce_out + u * a.reduce_stride + c, acc);
        } else {
          AdamRow4(T, slot, c, acc, write, st);
        }
      } else {
        for (uint32_t c0 = 0; c0 < dim; c0 += kWave) {
          const uint32_t c = c0 + lig;
          const bool active = c < dim;
          float acc = 0.f;
          for (uint32_t base = sb; base < se; base += kWave) {
            const uint32_t cnt = min(kWave, se - base);
            const uint64_t my = lig < cnt ? a.rs[base + lig] : 0ull;
            for (uint32_t k = 0; k < cnt; ++k) {
              const uint64_t w = __shfl(my, int(k), int(kWave));
              const uint32_t ref = uint32_t(w);
              const float s = __uint_as_float(uint32_t(w >> 32));
              const bool in = ref_ok(w);
              if (!in) ok = false;
              const float* src = s_grad[ref >> kRefRowBits] +
                                 uint64_t(ref & ((1u << kRefRowBits) - 1)) * dim;
              const float x = active && in ? LoadF(src + c) : 0.f;
              acc = acc + x * s;
            }
          }
          if (!ok) st.err |= EPS_HIP_STATUS_BAD_INDEX;
          if (!active || !ok) continue;
          if (a.reduce) {
            if (!Finite(acc)) st.err |= EPS_HIP_STATUS_REDUCE_OVERFLOW;
            a.reduce_out[u * a.reduce_stride + c] = acc;
          } else {
            AdamRow1(T, slot, c, acc, write, st);
          }
        }
      }
    }
    __syncthreads();
  }
  FinishBlock(st, ctrl, a.bounds, write && !a.reduce);
}

// ---------------------------------------------------------------------------
// Vector-class update (dim % 4 == 0, dim <= 256).  Two kernels:
//
//  * HotSliceKernel: rows with more than kLongRefs references (listed at
//    prepare time).  Work unit = (hot row, kSlice-column slice); a block
//    works through a stream of units chunk by chunk (64 references; 256 for
//    16-column units, so a chunk's tile holds the same 4,096 products).
//    Wave 0 adds: lane c < kSlice owns column col0 + c, adds the chunk's
//    products in reference order (one dependent add per reference) and
//    applies Adam after the unit's last chunk.  Waves 1..kProducers produce:
//    producer p loads the gradient rows of every kProducers-th chunk (16
//    contiguous bytes per lane), multiplies them by their scales and stores
//    the products into one of kHotRing LDS tiles [column][reference], with
//    the unit's w, m, v when the chunk is its last.  Tiles change hands
//    through two LDS counters per tile (staged / added), so the waves never
//    meet at a block barrier, and each producer keeps two chunks of rows in
//    flight (one of the longer 16-column chunks).  For very long rows the slices are narrow (32 columns) so that a
//    hot row's chain data spreads over several CUs: a block's producers then
//    move half of a 64-column chunk's bytes through their CU per chunk, and
//    the adding wave's serial chain, not the CU's memory pipeline, sets the
//    rate; a 32-column slice of a reference is one whole 128-byte line, so
//    no line is fetched for part of its bytes.  Small pushes with very long
//    rows (their gradient rows stay in the caches) take 16-column slices.
//  * RowRunKernel: every other row.  A block owns a window of sorted
//    positions (RunPositions: 256, or 128 / 64 for 32- / 64-lane groups, so
//    every group has a few rows per window whatever the width); it stages
//    their keys and reference words (plus kLongRefs positions of look-ahead)
//    in LDS with coalesced loads, finds the segment heads with a ballot, and a
//    group of G = dim/4 lanes per row (lane = 4 columns) loads the row's w, m,
//    v together with its gradient rows, sums them in order and applies Adam.
constexpr uint32_t kHotBlock = 256;                       // threads of a hot-row block
constexpr uint32_t kHotRing = 4;                          // chunks staged in LDS per block
constexpr uint32_t kUnitCache = 512;                      // unit headers a block stages in LDS
// Shape of a hot-row unit of kS columns (16, 32 or 64) in chunks of kC
// references (kS * kC = 4,096 or fewer products a tile): lanes per reference
// in a producer's row load, references per row load, row loads per producer
// lane per chunk, reference words per producer lane per chunk, floats per
// tile row (one column), and the parts the adding wave reads a tile in (of
// kPart references: 32 for 16-column units, whose 256-reference chunks would
// otherwise need more registers than the kernel has, 64 for the others).
template <uint32_t kS, uint32_t kC>
struct HotShape {
  static constexpr uint32_t kQuads = kS / 4;
  static constexpr uint32_t kRefsPerLoad = kWave / kQuads;
  static constexpr uint32_t kLoads = kC / kRefsPerLoad;
  static constexpr uint32_t kWords = kC / kWave;
  static constexpr uint32_t kPitch = kC + 4;
  static constexpr uint32_t kPart = kS < 32 ? kWave / 2 : kWave;
  // Own chunks each producer keeps in flight: two (four measured no faster,
  // and for the HBM-bound chains of 4 x 8.4 M references three or four made
  // the step 9.8 -> 11.3-11.7 ms), one for 16-column units, whose chunks of
  // 256 references keep as many bytes in flight and leave the registers for
  // their longer reference lists.
  static constexpr uint32_t kDepth = kS < 32 ? 1 : 2;
  static constexpr uint32_t kParts = kC / kPart;
  static_assert(kC % kWave == 0 && kS <= kWave && kWave % kQuads == 0 && kLoads % 4 == 0 &&
                    kLoads <= 16 && kS * kC <= kWave * kWave,
                "hot-row tile shape");
};
constexpr uint32_t kProducers = kHotBlock / kWave - 1;

// Sorted positions per row-run window for groups of 2^log2g lanes: about 5
// rows per group at the usual ~3 references per row.  Wider groups take
// narrower windows, so a class of wide rows still spreads over many blocks.
constexpr uint32_t RunPositions(uint32_t log2g) { return log2g <= 4 ? 256u : (log2g == 5 ? 128u : 64u); }
constexpr uint32_t kRunPositions = RunPositions(2);  // the widest window
static_assert(kRunPositions <= kBlock, "one thread per staged position finds the row heads");
constexpr uint32_t kRefBatch = 4;                       // gradient rows in flight per group

struct VecArgs {
  TableDesc t[EPS_HIP_MAX_TABLES];   // by key index
  const float* grad[EPS_HIP_MAX_FEATURES];
  uint64_t grad_rows[EPS_HIP_MAX_FEATURES];
  const uint32_t* keys;
  const uint64_t* rs;
  const HotEntry* hot;
  Control* ctrl;
  Bounds* bounds;
  GuardScalars gs;
  uint32_t row_bits, cls, role, slice_bits, hot_capacity, tables, features;
  uint32_t n;           // sorted positions of the push (hot-row entries are clamped to them)
  uint32_t spin_limit;  // polls of a hot-row hand-over wait (0: give up at once)
  uint32_t class_block[kClasses], class_grid[kClasses];  // RowRunClassesKernel's blocks per class
};
static_assert(sizeof(VecArgs) <= 4096, "update arguments fit the kernel-argument segment");

// Position of (column c, reference r) in a hot-row tile of kPitch floats a
// column.  Groups of four references are rotated by the column's 16-column
// group (XOR; the identity for slices of 16 columns), so a producer's stores
// of one row load hit distinct banks, and the adding wave's 16-byte reads of
// four consecutive references stay aligned.
template <uint32_t kPitch>
__device__ __forceinline__ uint32_t TileAt(uint32_t c, uint32_t r) {
  return c * kPitch + 4u * ((r >> 2) ^ (c >> 4)) + (r & 3u);
}

__device__ __forceinline__ const float* RefSource(const float* const* grad, uint64_t word,
                                                  uint32_t dim, uint32_t col, float& scale) {
  const uint32_t ref = uint32_t(word);
  scale = __uint_as_float(uint32_t(word >> 32));
  return grad[ref >> kRefRowBits] + uint64_t(ref & ((1u << kRefRowBits) - 1)) * dim + col;
}

// Copies the per-launch tables to LDS and decides whether this launch writes;
// returns false when it has nothing to do (uniform over the block).
template <uint32_t kThreads = kBlock>
__device__ __forceinline__ bool VecPrologue(const VecArgs& a, TableDesc* s_t, const float** s_grad,
                                            uint32_t* s_mode, bool& write, uint64_t* s_rows) {
  CopyWords<kThreads>(s_t, a.t, sizeof(a.t));
  CopyWords<kThreads>(s_grad, a.grad, sizeof(a.grad));
  CopyWords<kThreads>(s_rows, a.grad_rows, sizeof(a.grad_rows));
  return LaunchGate(a.ctrl, s_t, a.gs, a.role, s_mode, write);
}

// One chunk of a hot work unit: positions [cbase, cbase + chunk) of the
// row whose references are the sorted positions [start, end), for the kSlice
// columns from col0.  `ok` is false past the stream's last unit.  Every field
// is the same in all lanes of a wavefront.
struct HotSlot {
  uint32_t start, end, key, col0, cbase;
  bool ok;
};

// A producer's loads of one chunk in flight.  Row load k brings columns
// 4*quad .. 4*quad+3 of reference kHotRefsPerLoad*k + sub, with its scale;
// wmv is lane l's column of the unit's w, m, v (used when the chunk ends its
// unit).
template <uint32_t kS, uint32_t kC>
struct HotRows {
  HotSlot c;
  float4 x[HotShape<kS, kC>::kLoads];
  float s[HotShape<kS, kC>::kLoads];
  float wmv[3];
};

// A producer's row pointers and scales of one chunk, staged in LDS in the
// order the row loads use them: entry [sub][k] is reference
// kHotRefsPerLoad*k + sub, so a lane reads its kHotLoads pointers and scales
// with a few 16-byte reads.
template <uint32_t kS, uint32_t kC>
struct HotRefs {
  const float* src[HotShape<kS, kC>::kRefsPerLoad][HotShape<kS, kC>::kLoads];
  float scale[HotShape<kS, kC>::kRefsPerLoad][HotShape<kS, kC>::kLoads];
};

// s_waitcnt operand that waits for LDS (and scalar memory) accesses only:
// vmcnt and expcnt at their maxima, lgkmcnt 0.
constexpr int kLgkmZero = 0xC07F;

// Waits until the LDS counter reaches `target` (all lanes read the same word).
// Returns false on a timeout: a wait that has not been satisfied after `limit`
// polls marks the push failed and stops waiting, so a block always finishes
// (limit 0: every wait times out at once, the host-driven test of that path).
__device__ __forceinline__ bool WaitCounter(const uint32_t* counter, uint32_t target, uint32_t sleep,
                                            uint32_t limit) {
  if (limit == 0) return false;
  for (uint32_t spins = 0;; ++spins) {
    const uint32_t v = uint32_t(__builtin_amdgcn_readfirstlane(
        int(__hip_atomic_load(counter, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP))));
    if (v >= target) break;
    if (spins >= limit) return false;
    if (sleep) __builtin_amdgcn_s_sleep(1);
  }
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
  return true;
}

// Publishes `value` after this wave's earlier LDS accesses.
__device__ __forceinline__ void PostCounter(uint32_t* counter, uint32_t value) {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  if ((threadIdx.x & (kWave - 1)) == 0)
    __hip_atomic_store(counter, value, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

template <uint32_t kSlice, uint32_t kChunk>
__global__ void __launch_bounds__(kHotBlock) HotSliceKernel(VecArgs a) {
  using Shape = HotShape<kSlice, kChunk>;
  constexpr uint32_t kHotQuads = Shape::kQuads;
  constexpr uint32_t kHotRefsPerLoad = Shape::kRefsPerLoad;
  constexpr uint32_t kHotLoads = Shape::kLoads;
  constexpr uint32_t kPitch = Shape::kPitch;
  constexpr uint32_t kPart = Shape::kPart;
  constexpr uint32_t kParts = Shape::kParts;
  constexpr uint32_t kDepth = Shape::kDepth;
  __shared__ TableDesc s_t[EPS_HIP_MAX_TABLES];
  __shared__ const float* s_grad[EPS_HIP_MAX_FEATURES];
  __shared__ __align__(16) float s_tile[kHotRing][kSlice * kPitch];
  __shared__ float s_wmv[kHotRing][3][kSlice];
  __shared__ __align__(16) HotRefs<kSlice, kChunk> s_ref[kProducers];
  // ready[t]: chunks staged in tile t so far; used[t]: chunks added from it.
  __shared__ uint32_t s_ready[kHotRing], s_used[kHotRing];
  __shared__ uint4 s_unit[kUnitCache];  // {start, end, key, col0} of the block's first units
  __shared__ uint32_t s_mode;
  // Set when a hot-row entry, key or reference names nothing of the push (a
  // damaged workspace): the block writes nothing from then on.
  __shared__ uint32_t s_bad;
  __shared__ uint64_t s_rows[EPS_HIP_MAX_FEATURES];  // gradient rows per feature
  bool write = false;
  if (!VecPrologue<kHotBlock>(a, s_t, s_grad, &s_mode, write, s_rows)) return;
  if (threadIdx.x < kHotRing) {
    s_ready[threadIdx.x] = 0;
    s_used[threadIdx.x] = 0;
  }
  if (threadIdx.x == 0) s_bad = 0;
  Control* ctrl = a.ctrl;
  const uint32_t lane = threadIdx.x & (kWave - 1);
  const uint32_t wave = uint32_t(__builtin_amdgcn_readfirstlane(int(threadIdx.x / kWave)));
  RowStats st;
  __syncthreads();
  // XCD x takes its hot-row lists: the hot rows of the x-th eighth of the
  // sorted positions, whose gradient rows the row runs of that XCD also read.
  // Work units are (row, slice) in list order, longest rows first.  Units of
  // the first list (rows of 65,536 or more references) each get a block of
  // their own, when there are fewer of them than the XCD has blocks: one such
  // unit can take longer than all the shorter units spread over the other
  // blocks (4 x 8.4 M references: 15,200 chunks vs ~1,800 a block), so its
  // block takes nothing else.  The other units are dealt to the remaining
  // blocks in snake order (round r goes left to right when r is even, right
  // to left when odd), so the per-block totals stay close.
  const uint32_t xcd = blockIdx.x % kXcds;
  const uint32_t xcd_blocks = gridDim.x / kXcds;
  const uint32_t me = blockIdx.x / kXcds;
  const uint32_t slice_mask = (1u << a.slice_bits) - 1;
  uint32_t bucket_end[kHotBuckets];
  uint32_t units = 0;
#pragma unroll
  for (uint32_t b = 0; b < kHotBuckets; ++b) {
    const uint32_t count = uint32_t(__builtin_amdgcn_readfirstlane(int(ctrl->long_count[xcd * kHotBuckets + b])));
    units += min(count, a.hot_capacity) << a.slice_bits;
    bucket_end[b] = units;
  }
  // The block's unit u of round r (units or more: none), and where its
  // hot-row entry lies.
  const uint32_t own = bucket_end[0] < xcd_blocks ? bucket_end[0] : 0u;  // blocks with a unit of their own
  const uint32_t shared = xcd_blocks - own, mine = me - own;
  auto unit_of = [&](uint32_t r) {
    if (me < own) return r == 0 ? me : units;
    return own + r * shared + ((r & 1) ? shared - 1 - mine : mine);
  };
  // An entry's positions, kept inside the push's sorted positions (start < end
  // <= n), so a damaged list can neither read past them nor run unbounded.
  auto sane = [&](uint32_t& start, uint32_t& end) {
    if (start < end && end <= a.n) return true;
    start = min(start, a.n - 1);
    end = min(max(end, start + 1), a.n);
    return false;
  };
  auto entry_of = [&](uint32_t u, uint32_t& col0) {
    uint32_t b = 0;
#pragma unroll
    for (uint32_t k = 0; k + 1 < kHotBuckets; ++k) b += u >= bucket_end[k];
    const uint32_t local = u - (b ? bucket_end[b - 1] : 0u);
    col0 = (local & slice_mask) * kSlice;
    return uint64_t(xcd * kHotBuckets + b) * a.hot_capacity + (local >> a.slice_bits);
  };
  // The headers of the block's first kUnitCache units are staged in LDS once,
  // so walking the stream costs each wave an LDS read per unit.  (A scalar
  // load per unit would stall every wave's next LDS wait until it returns:
  // scalar loads and LDS accesses share one wait counter.)  Later units, if
  // any, are read through the scalar cache.
  for (uint32_t r = threadIdx.x; r < kUnitCache; r += kHotBlock) {
    const uint32_t u = unit_of(r);
    if (u < units) {
      uint32_t col0;
      HotEntry e = a.hot[entry_of(u, col0)];
      if (!sane(e.start, e.end)) s_bad = 1;
      s_unit[r] = make_uint4(e.start, e.end, e.key, col0);
    }
  }
  __syncthreads();
  const auto* hot = reinterpret_cast<const __attribute__((address_space(4))) HotEntry*>(
      reinterpret_cast<uintptr_t>(a.hot));
  // The block's stream of chunks; every wave walks it the same way.
  uint32_t round = 0;
  HotEntry next_entry{0, 0, 0, 0};
  uint32_t next_col0 = 0;
  bool next_ok = false;
  auto fetch = [&]() {  // header of the block's next unit
    const uint32_t r = round++;
    const uint32_t u = unit_of(r);
    next_ok = u < units;  // unit indices grow with the round: past the end stays past
    if (!next_ok) return;
    if (r < kUnitCache) {
      const uint4 e = s_unit[r];
      next_entry = HotEntry{e.x, e.y, e.z, 0u};
      next_col0 = e.w;
      return;
    }
    const auto& e = hot[entry_of(u, next_col0)];
    next_entry = HotEntry{e.start, e.end, e.key, 0u};
    if (!sane(next_entry.start, next_entry.end)) s_bad = 1;
  };
  auto take = [&]() {  // the next unit's first chunk; slices past a row's dimension are skipped
    for (;;) {
      HotSlot t{next_entry.start, next_entry.end, next_entry.key, next_col0, next_entry.start, next_ok};
      const uint32_t dim = uint32_t(__builtin_amdgcn_readfirstlane(
          int(s_t[min(next_entry.key >> a.row_bits, a.tables - 1)].dim)));
      const bool usable = !next_ok || next_col0 < dim;
      fetch();
      if (usable) return t;
    }
  };
  auto after = [&](const HotSlot& c) {  // the chunk that follows c in the stream
    if (c.ok && c.cbase + kChunk < c.end) {
      HotSlot t = c;
      t.cbase += kChunk;
      return t;
    }
    return take();
  };
  // A hand-over wait timed out: this wave stops waiting, staging, adding and
  // writing, and the push reports a failure.
  bool stalled = false;

  if (wave == 0) {
    // The adding wave: chunk j is the (j / kHotRing)-th use of tile j % kHotRing.
    // Chunk j + 1's tile is read while chunk j is added, and the readiness
    // of chunk j + 2 is polled at the same time; scheduling barriers keep the
    // compiler from moving those LDS accesses (or their waits) before the adds.
    __builtin_amdgcn_s_setprio(2);
    fetch();
    HotSlot c = take();          // chunk j
    HotSlot cn = after(c);       // chunk j + 1
    HotSlot cnn = after(cn);     // chunk j + 2
    float acc = 0.f;
    // Part h (references kPart * h onwards) of chunk j's tile into x.  With
    // one part a chunk, lanes past the slice read nothing.  With several,
    // they read a copy of a slice column and drop it: every lane then writes
    // all of x, so no old contents of a buffer stay live from part to part
    // (which would make the compiler copy whole buffers).
    const uint32_t sl = lane % kSlice;
    auto read_part = [&](uint32_t j, uint32_t h, float4* x) {
      const float* tile = s_tile[j % kHotRing];
      if (kParts > 1 || lane < kSlice) {
#pragma unroll
        for (uint32_t g = 0; g < kPart / 4; ++g)
          x[g] = *reinterpret_cast<const float4*>(tile + TileAt<kPitch>(sl, kPart * h + 4 * g));
      }
    };
    auto ready = [&](uint32_t j) {
      if (!stalled && !WaitCounter(&s_ready[j % kHotRing], j / kHotRing + 1, 0, a.spin_limit)) stalled = true;
    };
    // Adds chunk j (chunk c) part by part: part h is in x for even h and in y
    // for odd h, and each part's adds overlap the reads of the next part (of
    // chunk j + 1's first part after the last), which go to the other buffer.
    // So a chunk of an even number of parts starts and ends in x.  The
    // hand-over (tile release, readiness poll, walk to the next chunk) comes
    // once per chunk, whatever its length.  With several parts a chunk, the
    // next tile is read after the stream's last chunk all the same (plain LDS
    // reads, dropped), for the same reason.
    auto add = [&](uint32_t j, float4* x, float4* y) {
      const uint32_t t = j % kHotRing;
      float w = 0.f, m = 0.f, v = 0.f;
      uint32_t peek = 0;
#pragma unroll
      for (uint32_t h = 0; h < kParts; ++h) {
        const float4* cur = h % 2 ? y : x;
        float4* nxt = h % 2 ? x : y;
        // cur arrived during the previous adds.  Wait for it here, before more
        // reads are issued: the LDS counter tracks at most 15 accesses, so a
        // wait placed after the next part's 16 reads would wait for those too.
        __builtin_amdgcn_s_waitcnt(kLgkmZero);
        __builtin_amdgcn_sched_barrier(0);
        if (h + 1 < kParts) {
          read_part(j, h + 1, nxt);
        } else {
          w = s_wmv[t][0][sl];
          m = s_wmv[t][1][sl];
          v = s_wmv[t][2][sl];
          peek = __hip_atomic_load(&s_ready[(j + 2) % kHotRing], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
          if (kParts > 1 || cn.ok) read_part(j + 1, 0, nxt);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (uint32_t g = 0; g < kPart / 4; ++g) {
          acc = acc + cur[g].x;
          acc = acc + cur[g].y;
          acc = acc + cur[g].z;
          acc = acc + cur[g].w;
        }
        // With several parts, each part's sum is taken here: otherwise the
        // compiler sinks every part's adds below the last part's reads, which
        // then holds all the chunk's values in registers at once.
        if constexpr (kParts > 1) asm volatile("" : "+v"(acc));
        __builtin_amdgcn_sched_barrier(0);
      }
      // Tile t is free once chunk j's values and w, m, v are read: they were
      // read before tile j + 1's reads, and a wavefront's LDS accesses are
      // performed in order, so the counter store needs no wait for the reads
      // still in flight (the wavefront-scope fence keeps the compiler from
      // moving the reads after it).
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
      if (lane == 0)
        __hip_atomic_store(&s_used[t], j / kHotRing + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      __builtin_amdgcn_sched_barrier(0);
      if (c.cbase + kChunk >= c.end) {  // the unit's last chunk
        const KeyParts kp = SplitKey(c.key, a.row_bits);
        const TableDesc& T = s_t[min(kp.table, a.tables - 1)];
        if (!KeyInRange(kp, a.tables, T.rows)) s_bad = 1;
        if (lane < kSlice && c.col0 + lane < T.dim && !stalled) {
          AdamElement(T, acc, w, m, v, st);
          if (write && !s_bad) {
            float* row = T.state + uint64_t(kp.slot) * T.dim * 3 + c.col0 + lane;
            StoreF(row, w); StoreF(row + T.dim, m); StoreF(row + 2 * T.dim, v);
          }
        }
        acc = 0.f;
      }
      // Chunk j + 2 (if any) must be staged before the next call reads it.
      if (cnn.ok && uint32_t(__builtin_amdgcn_readfirstlane(int(peek))) < (j + 2) / kHotRing + 1)
        ready(j + 2);
      else
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
      c = cn;
      cn = cnn;
      cnn = after(cnn);
    };
    float4 xa[kPart / 4], xb[kPart / 4];
    if (c.ok) {
      ready(0);
      read_part(0, 0, xa);
      if (cn.ok) ready(1);
    }
    for (uint32_t j = 0; c.ok && !stalled; j += 2) {
      add(j, xa, xb);
      if (!c.ok || stalled) break;
      if constexpr (kParts % 2 == 1)
        add(j + 1, xb, xa);
      else
        add(j + 1, xa, xb);
    }
  } else {
    // Producer p stages chunks p, p + kProducers, ... (its own chunks, counted
    // by o).  At own chunk o it stages rows(o), decodes the words of o + D
    // into its LDS reference slots, loads the words of o + 2D and then the
    // rows of o + D (D = kDepth).  Loads complete in issue order, so each wait
    // waits only for what it needs.  Every chunk issues the same loads, also
    // past the stream's end (then from the start of the reference words, never
    // used), so the number of loads between any two points is fixed.
    const uint32_t p = wave - 1;
    const uint32_t quad = lane % kHotQuads, sub = lane / kHotQuads;
    const float* idle = reinterpret_cast<const float*>(a.rs);
    HotRefs<kSlice, kChunk>& slots = s_ref[p];
    fetch();
    HotSlot cur = take();  // cursor over the stream, at chunk jc
    uint32_t jc = 0, total = cur.ok ? ~0u : 0u;
    auto advance = [&](uint32_t by) {
      for (uint32_t i = 0; i < by; ++i) {
        cur = after(cur);
        ++jc;
        if (!cur.ok && total == ~0u) total = jc;
      }
    };
    // Reference words of one chunk in flight (lane l: references l, l + 64, ...).
    struct Words {
      HotSlot c;
      uint64_t word[Shape::kWords];
    };
    HotSlot dc{};  // chunk whose references are in the LDS slots
    auto load_words = [&](Words& w) {
      w.c = cur;
#pragma unroll
      for (uint32_t k = 0; k < Shape::kWords; ++k) {
        const uint32_t pos = cur.ok ? min(cur.cbase + kWave * k + lane, cur.end - 1) : 0u;  // end <= n (sane)
        w.word[k] = a.rs[pos];
      }
    };
    // Lane l decodes the words of references l, l + 64, ...: their gradient
    // rows (from the slice's first column) and scales.
    auto decode = [&](const Words& w) {
      const HotSlot& wc = w.c;
      dc = wc;
      const TableDesc& T = s_t[min(wc.key >> a.row_bits, a.tables - 1)];
#pragma unroll
      for (uint32_t k = 0; k < Shape::kWords; ++k) {
        const uint32_t r = kWave * k + lane;
        const RefParts rp = SplitRef(w.word[k]);
        const bool ref_ok = RefInRange(rp, a.features, s_rows[min(rp.feature, a.features - 1)]);
        if (wc.ok && !ref_ok) s_bad = 1;
        float scale;
        const float* src = RefSource(s_grad, w.word[k], T.dim, wc.col0, scale);
        slots.src[r % kHotRefsPerLoad][r / kHotRefsPerLoad] = wc.ok && ref_ok ? src : idle;
        slots.scale[r % kHotRefsPerLoad][r / kHotRefsPerLoad] = scale;
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
    };
    // Lanes whose columns lie past the row's dimension read the slice's first
    // columns; their products are never stored by the adding wave.
    auto load_rows = [&](HotRows<kSlice, kChunk>& r) {
      r.c = dc;
      const KeyParts kp = SplitKey(dc.key, a.row_bits);
      const TableDesc& T = s_t[min(kp.table, a.tables - 1)];
      const bool key_ok = KeyInRange(kp, a.tables, T.rows);
      const uint32_t dim = T.dim;
      const uint32_t off = dc.col0 + 4 * quad < dim ? 4 * quad : 0u;
      const uint32_t step = dc.ok ? off : 0u;
      const float* src[kHotLoads];
#pragma unroll
      for (uint32_t k = 0; k < kHotLoads; k += 2) {
        const uint4 two = *reinterpret_cast<const uint4*>(&slots.src[sub][k]);
        src[k] = reinterpret_cast<const float*>(uint64_t(two.x) | (uint64_t(two.y) << 32));
        src[k + 1] = reinterpret_cast<const float*>(uint64_t(two.z) | (uint64_t(two.w) << 32));
      }
#pragma unroll
      for (uint32_t k = 0; k < kHotLoads; k += 4) {
        const float4 four = *reinterpret_cast<const float4*>(&slots.scale[sub][k]);
        r.s[k] = four.x; r.s[k + 1] = four.y; r.s[k + 2] = four.z; r.s[k + 3] = four.w;
      }
#pragma unroll
      for (uint32_t k = 0; k < kHotLoads; ++k) r.x[k] = Load4(src[k] + step);
      const uint32_t wcol = dc.col0 + (lane < kSlice && dc.col0 + lane < dim ? lane : 0u);
      const float* row = dc.ok && key_ok ? T.state + uint64_t(kp.slot) * dim * 3 + wcol : idle;
      const uint32_t ms = dc.ok && key_ok ? dim : 0u;
      r.wmv[0] = LoadF(row); r.wmv[1] = LoadF(row + ms); r.wmv[2] = LoadF(row + 2 * ms);
    };
    auto stage = [&](const HotRows<kSlice, kChunk>& r, uint32_t j) {
      const uint32_t t = j % kHotRing;
      if (!stalled && !WaitCounter(&s_used[t], j / kHotRing, 1, a.spin_limit)) stalled = true;
      if (stalled) return;  // nothing more is staged
      // Load k brings columns 4*quad .. 4*quad+3 of reference
      // kHotRefsPerLoad*k + sub; each lands at TileAt(column, reference).
      float* tile = s_tile[t];
      if (r.c.cbase + kChunk <= r.c.end) {  // every reference inside the row
#pragma unroll
        for (uint32_t k = 0; k < kHotLoads; ++k) {
          const float sv = r.s[k];
          float* q = tile + TileAt<kPitch>(4 * quad, kHotRefsPerLoad * k + sub);
          q[0] = r.x[k].x * sv;
          q[kPitch] = r.x[k].y * sv;
          q[2 * kPitch] = r.x[k].z * sv;
          q[3 * kPitch] = r.x[k].w * sv;
        }
      } else {  // references past the row's end add -0.0f, the identity
#pragma unroll
        for (uint32_t k = 0; k < kHotLoads; ++k) {
          const bool in = r.c.cbase + kHotRefsPerLoad * k + sub < r.c.end;
          const float sv = r.s[k];
          float* q = tile + TileAt<kPitch>(4 * quad, kHotRefsPerLoad * k + sub);
          q[0] = in ? r.x[k].x * sv : -0.f;
          q[kPitch] = in ? r.x[k].y * sv : -0.f;
          q[2 * kPitch] = in ? r.x[k].z * sv : -0.f;
          q[3 * kPitch] = in ? r.x[k].w * sv : -0.f;
        }
      }
      if (lane < kSlice) {
        s_wmv[t][0][lane] = r.wmv[0];
        s_wmv[t][1][lane] = r.wmv[1];
        s_wmv[t][2][lane] = r.wmv[2];
      }
      PostCounter(&s_ready[t], j / kHotRing + 1);
    };
    // kDepth own chunks of rows and of reference words in flight.  The
    // prologue leaves the loads in the loop's own order (words(D), rows(0),
    // words(D+1), rows(1), ...), so the compiler's load waits inside the loop
    // can be exact.
    HotRows<kSlice, kChunk> rows[kDepth];
    Words words[kDepth];
    advance(p);  // own chunk 0
#pragma unroll
    for (uint32_t k = 0; k < kDepth; ++k) {  // words(0 .. D-1)
      load_words(words[k]);
      advance(kProducers);
    }
#pragma unroll
    for (uint32_t k = 0; k < kDepth; ++k) {  // words(D + k), then rows(k) from the slots of own chunk k
      decode(words[k]);
      load_words(words[k]);
      advance(kProducers);
      load_rows(rows[k]);
    }
    // Own chunk o (chunk j = p + kProducers*o), buffers b = o % D: stage
    // rows(o), decode words(o + D), load words(o + 2D) and rows(o + D).
    // Words and rows both get D own chunks to arrive (the decode needs no
    // wait of its own: its words were issued before the rows the stage
    // waited for).  D own chunks per pass keep the buffers static.
    auto own = [&](HotRows<kSlice, kChunk>& r, Words& w, uint32_t j) {
      stage(r, j);
      decode(w);
      load_words(w);
      advance(kProducers);
      load_rows(r);
    };
    uint32_t j = p;
    for (; j + (kDepth - 1) * kProducers < total; j += kDepth * kProducers) {  // one exit: every part runs
#pragma unroll
      for (uint32_t k = 0; k < kDepth; ++k) own(rows[k], words[k], j + k * kProducers);
    }
#pragma unroll
    for (uint32_t k = 0; k + 1 < kDepth; ++k)
      if (j + k * kProducers < total) stage(rows[k], j + k * kProducers);
  }
  if (stalled) st.err |= EPS_HIP_STATUS_STALLED;
  __syncthreads();
  if (s_bad) st.err |= EPS_HIP_STATUS_BAD_INDEX;
  FinishBlock<kHotBlock / kWave>(st, ctrl, a.bounds, write);
}

// LDS of a row-run block, sized for the widest window.
struct RunShared {
  uint32_t key[kRunPositions + kLongRefs + 1];  // key[i + 1] = key at position p0 + i
  const float* src[kRunPositions + kLongRefs];  // gradient row of position p0 + i
  float scale[kRunPositions + kLongRefs];
  uint32_t heads[kRunPositions];
  uint32_t wave_heads[kBlock / kWave];
  uint32_t next;  // next unclaimed row (head index) of the window
  uint32_t bad;
};

// The rows of dimension class `cls` (groups of 2^kLog2G lanes), for block
// `block` of the `grid` blocks the class has.
template <uint32_t kLog2G>
__device__ __forceinline__ void RowRuns(const VecArgs& a, RunShared& sh, const TableDesc* s_t,
                                        const float* const* s_grad, const uint64_t* s_rows, uint32_t cls,
                                        uint32_t block, uint32_t grid, bool write, RowStats& st) {
  constexpr uint32_t G = 1u << kLog2G;
  constexpr uint32_t ngroups = kBlock / G;
  constexpr uint32_t kWindow = RunPositions(kLog2G);
  constexpr uint32_t kStaged = kWindow + kLongRefs;
  static_assert(kStaged <= kRunPositions + kLongRefs, "row-run window fits its LDS");
  Control* ctrl = a.ctrl;
  // Safe address for reads a damaged workspace would point elsewhere: the
  // control block and what follows it (far more than a row of 3 x 256 floats).
  const float* safe = reinterpret_cast<const float*>(a.ctrl);
  // The class's sorted positions, from the workspace: kept inside the push's
  // positions, so a damaged workspace cannot send the staging reads past them.
  const uint32_t first = ctrl->class_start[cls], last = ctrl->class_start[cls + 1];
  const uint32_t end = min(last, a.n), begin = min(first, end);
  const uint32_t row_mask = (1u << a.row_bits) - 1;
  const uint32_t lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  const uint32_t lig = threadIdx.x & (G - 1), gid = threadIdx.x >> kLog2G;
  const uint32_t c = lig * 4;
  // The class's positions are cut into kXcds contiguous ranges, one per XCD
  // (the class's blocks start at a multiple of kXcds and number a multiple of
  // it, and blocks reach the XCDs round robin): the gradient rows a range
  // references then come from a few features and stay in that XCD's L2 for
  // all their references.  Rows that straddle a cut belong to the range
  // holding their first position.
  const uint32_t xcd = block % kXcds, per_xcd = grid / kXcds;
  const uint32_t span = ((end - begin + kXcds - 1) / kXcds + kWindow - 1) / kWindow * kWindow;
  const uint32_t xbegin = min(begin + xcd * span, end), xend = min(xbegin + span, end);
  for (uint32_t p0 = xbegin + (block / kXcds) * kWindow; p0 < xend; p0 += per_xcd * kWindow) {
    const uint32_t p1 = min(p0 + kWindow, xend);
    const uint32_t lim = min(p1 + kLongRefs, end);
    const uint32_t staged = lim - p0;
    __syncthreads();  // previous iteration's readers are done
    // Stage keys and, per position, the gradient row it references and its
    // scale (one coalesced pass; the table and feature lookups happen here
    // once per position instead of once per lane).
    if (threadIdx.x == 0) {
      sh.key[0] = p0 > begin ? a.keys[p0 - 1] : ~a.keys[p0];
      sh.next = ngroups;
    }
    for (uint32_t i = threadIdx.x; i < staged; i += kBlock) {
      const uint32_t key = a.keys[p0 + i];
      const uint64_t word = a.rs[p0 + i];
      sh.key[i + 1] = key;
      // A key or reference that names no table, slot, feature or gradient row
      // of the push (a damaged workspace) is read from a safe address instead,
      // and the block writes nothing from then on.
      const KeyParts kp = SplitKey(key, a.row_bits);
      const RefParts rp = SplitRef(word);
      const uint32_t ti = min(kp.table, a.tables - 1);
      const uint32_t fi = min(rp.feature, a.features - 1);
      const bool ok = KeyInRange(kp, a.tables, s_t[ti].rows) && RefInRange(rp, a.features, s_rows[fi]);
      float scale;
      const float* src = RefSource(s_grad, word, s_t[ti].dim, 0, scale);
      sh.src[i] = ok ? src : safe;
      sh.scale[i] = scale;
      if (!ok) sh.bad = 1;
    }
    __syncthreads();
    const bool window_ok = sh.bad == 0;
    const bool head = threadIdx.x < p1 - p0 && sh.key[threadIdx.x + 1] != sh.key[threadIdx.x];
    const uint64_t ballot = __ballot(head);
    if (lane == 0) sh.wave_heads[wave] = uint32_t(__popcll(ballot));
    __syncthreads();
    uint32_t before = 0;
    for (uint32_t w = 0; w < wave; ++w) before += sh.wave_heads[w];
    uint32_t nheads = 0;
    for (uint32_t w = 0; w < kBlock / kWave; ++w) nheads += sh.wave_heads[w];
    if (head) sh.heads[before + uint32_t(__popcll(ballot & ((1ull << lane) - 1)))] = threadIdx.x;
    __syncthreads();
    // Groups take rows in order from a shared counter (claimed at the top of
    // a row, used at its end), so a group held up by a row with many
    // references does not hold up the rows behind it.
    for (uint32_t h = gid; h < nheads;) {
      uint32_t claim = 0;
      if (lig == 0) claim = atomicAdd(&sh.next, 1u);
      const uint32_t sb = sh.heads[h];
      const uint32_t key = sh.key[sb + 1];
      // Hot rows (more than kLongRefs references) belong to HotSliceKernel.
      if (sb + kLongRefs < staged && sh.key[sb + kLongRefs + 1] == key) {
        h = uint32_t(__shfl(int(claim), 0, int(G)));
        continue;
      }
      uint32_t se = h + 1 < nheads ? sh.heads[h + 1] : p1 - p0;
      while (se < staged && sh.key[se + 1] == key) ++se;
      const TableDesc& T = s_t[min(key >> a.row_bits, a.tables - 1)];
      const uint32_t dim = T.dim;
      const bool active = c < dim;
      const uint32_t cl = active ? c : 0;  // inactive lanes read column 0 and drop it
      float* row = window_ok ? T.state + uint64_t(key & row_mask) * dim * 3 : const_cast<float*>(safe);
      const float4 w0 = Load4Stream(row + cl), m0 = Load4Stream(row + dim + cl),
                   v0 = Load4Stream(row + 2 * dim + cl);
      float4 g = make_float4(0.f, 0.f, 0.f, 0.f);
      // Every slot of a batch loads (slots past the row repeat its last
      // reference, an in-bounds row of the same table); only real references
      // are added, in order.  The first batch is straight-line code so its
      // loads go out together with w, m and v; longer rows loop.
      auto batch = [&](uint32_t j0) {
        float4 x[kRefBatch];
        float s[kRefBatch];
#pragma unroll
        for (uint32_t k = 0; k < kRefBatch; ++k) {
          const uint32_t j = min(j0 + k, se - 1);
          s[k] = sh.scale[j];
          x[k] = Load4(sh.src[j] + cl);
        }
#pragma unroll
        for (uint32_t k = 0; k < kRefBatch; ++k) {
          float4 t = g;
          Accumulate4(t, x[k], s[k]);
          if (j0 + k < se) g = t;
        }
      };
      batch(sb);
      for (uint32_t j0 = sb + kRefBatch; j0 < se; j0 += kRefBatch) batch(j0);
      if (active) {
        float4 w = w0, m = m0, v = v0;
        if (T.bounded) {
          AdamElement<true>(T, g.x, w.x, m.x, v.x, st);
          AdamElement<true>(T, g.y, w.y, m.y, v.y, st);
          AdamElement<true>(T, g.z, w.z, m.z, v.z, st);
          AdamElement<true>(T, g.w, w.w, m.w, v.w, st);
        } else {
          AdamElement<false>(T, g.x, w.x, m.x, v.x, st);
          AdamElement<false>(T, g.y, w.y, m.y, v.y, st);
          AdamElement<false>(T, g.z, w.z, m.z, v.z, st);
          AdamElement<false>(T, g.w, w.w, m.w, v.w, st);
        }
        if (write && window_ok) {
          Store4Stream(row + c, w);
          Store4Stream(row + dim + c, m);
          Store4Stream(row + 2 * dim + c, v);
        }
      }
      h = uint32_t(__shfl(int(claim), 0, int(G)));
    }
  }
}

// Seven waves per SIMD (72 registers) where that needs no spill: more rows'
// loads in flight per CU.
template <uint32_t kLog2G>
__global__ void __launch_bounds__(kBlock) __attribute__((amdgpu_waves_per_eu(kLog2G == 2 || kLog2G == 6 ? 6 : 7)))
RowRunKernel(VecArgs a) {
  __shared__ TableDesc s_t[EPS_HIP_MAX_TABLES];
  __shared__ const float* s_grad[EPS_HIP_MAX_FEATURES];
  __shared__ RunShared sh;
  __shared__ uint32_t s_mode;
  __shared__ uint64_t s_rows[EPS_HIP_MAX_FEATURES];  // gradient rows per feature
  bool write = false;
  if (!VecPrologue(a, s_t, s_grad, &s_mode, write, s_rows)) return;
  RowStats st;
  if (threadIdx.x == 0) sh.bad = 0;
  __syncthreads();
  RowRuns<kLog2G>(a, sh, s_t, s_grad, s_rows, a.cls, blockIdx.x, gridDim.x, write, st);
  if (sh.bad) st.err |= EPS_HIP_STATUS_BAD_INDEX;
  FinishBlock(st, a.ctrl, a.bounds, write);
}

// Every vector class of a push in one launch: class c has the blocks
// [class_block[c], class_block[c] + class_grid[c]) (starts and counts are
// multiples of kXcds; absent classes have none), so the classes' rows run
// side by side instead of one launch (and its tail) after another.
__global__ void __launch_bounds__(kBlock) __attribute__((amdgpu_waves_per_eu(6)))
RowRunClassesKernel(VecArgs a) {
  __shared__ TableDesc s_t[EPS_HIP_MAX_TABLES];
  __shared__ const float* s_grad[EPS_HIP_MAX_FEATURES];
  __shared__ RunShared sh;
  __shared__ uint32_t s_mode;
  __shared__ uint64_t s_rows[EPS_HIP_MAX_FEATURES];
  bool write = false;
  if (!VecPrologue(a, s_t, s_grad, &s_mode, write, s_rows)) return;
  RowStats st;
  if (threadIdx.x == 0) sh.bad = 0;
  __syncthreads();
  uint32_t cls = 0;
#pragma unroll
  for (uint32_t c = 1; c + 1 < kClasses; ++c)
    if (a.class_grid[c] && blockIdx.x >= a.class_block[c]) cls = c;
  const uint32_t block = blockIdx.x - a.class_block[cls], grid = a.class_grid[cls];
  switch (cls) {
    case 0: RowRuns<2>(a, sh, s_t, s_grad, s_rows, 0, block, grid, write, st); break;
    case 1: RowRuns<3>(a, sh, s_t, s_grad, s_rows, 1, block, grid, write, st); break;
    case 2: RowRuns<4>(a, sh, s_t, s_grad, s_rows, 2, block, grid, write, st); break;
    case 3: RowRuns<5>(a, sh, s_t, s_grad, s_rows, 3, block, grid, write, st); break;
    default: RowRuns<6>(a, sh, s_t, s_grad, s_rows, 4, block, grid, write, st); break;
  }
  if (sh.bad) st.err |= EPS_HIP_STATUS_BAD_INDEX;
  FinishBlock(st, a.ctrl, a.bounds, write);
}

// ---------------------------------------------------------------------------
// Row driver: explicit unique rows (ApplyHost) or CSR references (ApplyCompact).
struct RowArgs {
  TableDesc t;
  const uint64_t* slots;
  const uint64_t* offsets;   // NULL: row r has exactly gradient row r (ApplyHost)
  const uint64_t* sources;
  const float* scales;
  const float* src;
  uint64_t rows;
  Control* ctrl;
  Bounds* bounds;
  GuardScalars gs;
  uint32_t log2g, vblocks, role;
};

template <bool kGeneric>
__global__ void __launch_bounds__(kBlock) RowUpdateKernel(RowArgs a) {
  __shared__ TableDesc s_t[1];
  __shared__ uint32_t s_mode;
  Control* ctrl = a.ctrl;
  if (threadIdx.x == 0) s_t[0] = a.t;
  bool write = false;
  if (!LaunchGate(ctrl, s_t, a.gs, a.role, &s_mode, write)) return;
  const TableDesc T = a.t;
  const uint32_t dim = T.dim;
  const uint32_t G = kGeneric ? kWave : (1u << a.log2g);
  const uint32_t lig = threadIdx.x & (G - 1);
  const uint32_t gid = threadIdx.x / G, ngroups = kBlock / G;
  RowStats st;
  for (uint32_t vb = blockIdx.x; vb < a.vblocks; vb += gridDim.x) {
    const uint64_t r = uint64_t(vb) * ngroups + gid;
    if (r >= a.rows) continue;
    const uint64_t slot = a.slots[r];
    if (!kGeneric) {
      const uint32_t c = lig * 4;
      const bool active = c < dim;
      float4 g;
      if (!a.offsets) {
        g = active ? Load4(a.src + r * dim + c) : make_float4(0.f, 0.f, 0.f, 0.f);
      } else {
        g = make_float4(0.f, 0.f, 0.f, 0.f);
        const uint64_t b = a.offsets[r], e = a.offsets[r + 1];
        for (uint64_t j = b; j < e; ++j) {
          const float s = a.scales[j];
          const float4 x = active ? Load4(a.src + a.sources[j] * dim + c) : make_float4(0.f, 0.f, 0.f, 0.f);
          Accumulate4(g, x, s);
        }
      }
      if (active) AdamRow4(T, slot, c, g, write, st);
    } else {
      for (uint32_t c = lig; c < dim; c += kWave) {
        float g;
        if (!a.offsets) {
          g = a.src[r * dim + c];
        } else {
          g = 0.f;
          for (uint64_t j = a.offsets[r]; j < a.offsets[r + 1]; ++j)
            g = g + a.src[a.sources[j] * dim + c] * a.scales[j];
        }
        AdamRow1(T, slot, c, g, write, st);
      }
    }
  }
  FinishBlock(st, ctrl, a.bounds, write);
}

// ---------------------------------------------------------------------------
TableDesc MakeTable(const eps_hip_table& t, const eps_hip_optimizer& o) {
  TableDesc d;
  d.state = t.state;
  d.rows = t.rows;
  d.dim = t.dim;
  d.beta1 = o.beta1;
  d.beta2 = o.beta2;
  d.omb1 = 1.0f - o.beta1;  // (1 - o.beta1) in float, lazy_adam.cpp:31
  d.omb2 = 1.0f - o.beta2;
  // lr_t in float exactly as lazy_adam.cpp:27 / cache_backend.cu:341.
  d.lr = o.learning_rate * std::sqrt(1 - o.beta2_power) / (1 - o.beta1_power);
  d.eps = o.epsilon;
  d.lo = o.bounded ? o.weight_min : -FLT_MAX;
  d.hi = o.bounded ? o.weight_max : FLT_MAX;
  d.bounded = o.bounded ? 1u : 0u;
  return d;
}

int CheckOptimizer(const eps_hip_optimizer& o) {
  // UpdateContext validation, src/cuda/cache_backend.cu:321-325.
  if (!(std::isfinite(o.learning_rate) && o.learning_rate > 0 && o.beta1_power >= 0 &&
        o.beta1_power < 1 && o.beta2_power >= 0 && o.beta2_power < 1))
    return Fail(EPS_HIP_INVALID_ARGUMENT, "invalid update context");
  if (o.bounded && !(std::isfinite(o.weight_min) && std::isfinite(o.weight_max) &&
                     o.weight_min <= o.weight_max))
    return Fail(EPS_HIP_INVALID_ARGUMENT, "invalid optimizer weight bounds");
  const float lr = o.learning_rate * std::sqrt(1 - o.beta2_power) / (1 - o.beta1_power);
  if (!std::isfinite(lr)) return Fail(EPS_HIP_INVALID_ARGUMENT, "optimizer learning-rate overflow");
  return EPS_HIP_OK;
}

uint32_t Log2G(uint32_t dim) {
  uint32_t log2g = 2;
  while ((1u << log2g) < dim / 4) ++log2g;
  return log2g;
}

// The gradient scan.  It always runs (one block at least), since its block 0
// takes the bounds snapshot the guard decides from; the decision itself is
// made by the first kernel of the update (DecideBlock).
int LaunchGuard(const GuardArgs& g, uint64_t blocks, hipStream_t s) {
  hipLaunchKernelGGL(GradMaxKernel, dim3(unsigned(std::max<uint64_t>(blocks, 1))), dim3(kBlock), 0, s, g);
  EPS_HIP_LAUNCHED("gradient guard");
  return EPS_HIP_OK;
}

uint64_t SpanBlocks(uint64_t count, SpanKind kind = kGradientSpan) {
  const uint64_t per = kind == kSortedSpan ? uint64_t(kBlock) * kSortedItems : uint64_t(kBlock) * kMaxItems * 4;
  return (count + per - 1) / per;
}

// The hot-row kernel's side stream and fork/join events, per calling thread
// and device (created on first use, default priority, never destroyed), so
// concurrent callers never share an event.
struct Overlap {
  hipStream_t side = nullptr;
  hipEvent_t fork = nullptr, join = nullptr;
};
int ThreadOverlap(Overlap** out) {
  constexpr int kDevices = 64;
  thread_local Overlap per_device[kDevices];
  int device = 0;
  EPS_HIP_TRY(Check(hipGetDevice(&device), "hipGetDevice"));
  if (device < 0 || device >= kDevices) return Fail(EPS_HIP_UNAVAILABLE, "device ordinal out of range");
  Overlap& o = per_device[device];
  if (!o.side) {
    EPS_HIP_TRY(Check(hipStreamCreateWithFlags(&o.side, hipStreamNonBlocking), "hot-row stream"));
    EPS_HIP_TRY(Check(hipEventCreateWithFlags(&o.fork, hipEventDisableTiming), "hot-row fork event"));
    EPS_HIP_TRY(Check(hipEventCreateWithFlags(&o.join, hipEventDisableTiming), "hot-row join event"));
  }
  *out = &o;
  return EPS_HIP_OK;
}

// The hot-row kernel runs beside the row kernels (on a side stream): its
// serial chains then overlap the row traffic instead of preceding it
// (measured on MI355X: 65,536 pairs on one table, 167 -> 133 us a push; 4 x
// 8.4 M references, 13.4 -> 11.6 ms; 26 tables of ~43,000 references with
// 64-column units on 256 blocks, 245 -> 236 us a step).  Pushes with a table
// of at least this many references take 32- or 16-column units on 512 blocks,
// so a very long row's chain data spreads over several CUs.
constexpr uint64_t kOverlapTableRefs = 1ull << 16;
constexpr uint32_t kFineSlice = 16, kNarrowSlice = 32, kWideSlice = 64;  // columns per hot-row unit
// References per hot-row chunk of each unit width.  16-column units take
// chunks of 256 references (a tile of 4,096 products, like a 64-column
// chunk), so their blocks hand a tile over (release, readiness poll, walk to
// the next chunk) once per 256 references instead of once per 64: 65,536
// pairs on one table, fused update 98-102 -> 84-91 us.  32-column units keep
// 64: with 128 the kernel needs 256 registers and 84 KB of LDS, one block per
// CU instead of two, and 4 x 8.4 M references lost (update 7.4-8.2 -> 8.1-8.3
// ms).
constexpr uint32_t kFineChunk = 256, kNarrowChunk = 64, kWideChunk = 64;
// Pushes with very long rows but fewer vector references than this take
// 16-column units (below).
constexpr uint64_t kFinePushRefs = 1ull << 18;

std::atomic<uint32_t> g_spin_limit{1u << 22};
uint32_t SpinLimit() { return g_spin_limit.load(std::memory_order_relaxed); }
// Whether this thread's pushes run the hot-row kernel on the side stream.
thread_local bool t_hot_row_overlap = true;

// Phases of a push (kPrimary: the fused update; kSecond: the checked apply)
// and kOneStream: every kernel on the caller's stream, the hot-row kernel
// before the row kernels (no side stream or event is created or used, so the
// push can be captured in a graph).
constexpr int kPrimary = 1, kSecond = 2, kOneStream = 4;
constexpr uint64_t kVectorGrid = 4096;  // persistent grid cap of the vector kernels
constexpr uint64_t kSecondGrid = 32;      // grid cap of the checked apply: it usually exits at
                                          // once, and a small grid launches faster
constexpr uint64_t kHotGrid = 512;      // two blocks per CU (LDS: four 17 KiB tiles per block)
// Blocks of the 64-column hot-row kernel beside the row kernels: enough to
// finish the hot rows well before the row kernels do, few enough to leave
// them most of the GPU (26 tables of ~43,000 references: 64 blocks 259 us a
// step of pull + push, 256 blocks 236, 512 blocks 240).
constexpr uint64_t kWideHotGrid = 256;

// A launch that also records `done` when the kernel completes (nullptr: a
// plain launch).  The event then rides on the kernel's own completion signal,
// with no marker packet after it in the stream.  For the join of the side
// stream: 26 tables of ~43,000 references, 0.2723 -> 0.2687 ms a step over six
// paired runs on one box (each faster than its pair), 0.2708 -> 0.2701 over
// four on another; 65,536 pairs on one table 0.111 -> 0.109 ms.
template <typename... Args>
void LaunchRecording(void (*kernel)(Args...), dim3 grid, dim3 block, hipStream_t s, hipEvent_t done,
                     Args... args) {
  if (done)
    hipExtLaunchKernelGGL(kernel, grid, block, 0, s, nullptr, done, 0, args...);
  else
    hipLaunchKernelGGL(kernel, grid, block, 0, s, args...);
}

template <uint32_t kLog2G>
int LaunchRowRun(unsigned grid, const VecArgs& a, hipStream_t s, hipEvent_t done) {
  LaunchRecording(RowRunKernel<kLog2G>, dim3(grid), dim3(kBlock), s, done, a);
  EPS_HIP_LAUNCHED("row update");
  return EPS_HIP_OK;
}

// Hot rows (any vector class) when `hot_slice`, else the other rows of class
// `cls`; `done` (if any) is recorded when the launch completes.
int LaunchVectorUpdate(uint32_t cls, uint32_t hot_slice, unsigned grid, const VecArgs& a, hipStream_t s,
                       hipEvent_t done = nullptr) {
  if (hot_slice) {
    if (hot_slice == kWideSlice)
      LaunchRecording(HotSliceKernel<kWideSlice, kWideChunk>, dim3(grid), dim3(kHotBlock), s, done, a);
    else if (hot_slice == kFineSlice)
      LaunchRecording(HotSliceKernel<kFineSlice, kFineChunk>, dim3(grid), dim3(kHotBlock), s, done, a);
    else
      LaunchRecording(HotSliceKernel<kNarrowSlice, kNarrowChunk>, dim3(grid), dim3(kHotBlock), s, done, a);
    EPS_HIP_LAUNCHED("hot row update");
    return EPS_HIP_OK;
  }
  switch (cls) {
    case 0: return LaunchRowRun<2>(grid, a, s, done);
    case 1: return LaunchRowRun<3>(grid, a, s, done);
    case 2: return LaunchRowRun<4>(grid, a, s, done);
    case 3: return LaunchRowRun<5>(grid, a, s, done);
    case 4: return LaunchRowRun<6>(grid, a, s, done);
    default: return Fail(EPS_HIP_INVALID_ARGUMENT, "no vector kernel for this dimension class");
  }
}

int RunSorted(const eps_hip_table* tables, const eps_hip_optimizer* optimizers, uint32_t table_count,
              const eps_hip_push_feature* features, uint32_t feature_count, const PushPlan& plan,
              const PushLayout& L, uint8_t* ws, bool reduce, const uint64_t* occ2u, float* out,
              uint64_t stride, Bounds* bounds, hipStream_t s, int phases) {
  FusedArgs a{};
  const bool in_b = plan.passes % 2 == 1;
  a.keys = reinterpret_cast<const uint32_t*>(ws + (in_b ? L.keys_b : L.keys_a));
  a.vals = reinterpret_cast<const uint32_t*>(ws + (in_b ? L.vals_b : L.vals_a));
  a.rs = reinterpret_cast<const uint64_t*>(ws + L.sorted_rs);
  a.occ2u = occ2u;
  a.reduce_out = out;
  a.reduce_stride = stride;
  a.ctrl = reinterpret_cast<Control*>(ws);
  a.bounds = bounds;
  a.row_bits = plan.row_bits;
  a.reduce = reduce ? 1 : 0;
  a.tables = table_count;
  a.features = feature_count;
  a.n = uint32_t(plan.occurrences);
  a.gs = GuardScalars{0, table_count};  // refs: the prepared valid count
  // The first kernel of the primary phase makes the guard decision.
  uint32_t role = kDecide;
  bool overlap = false;  // hot rows (on the side stream, joined before the checked apply)
  Overlap* ov = nullptr;
  for (uint32_t k = 0; k < table_count; ++k) {
    const uint32_t t = plan.table_of_key[k];
    eps_hip_optimizer o{};
    if (optimizers) o = optimizers[t];
    else { o.learning_rate = 1; o.beta1 = 0; o.beta2 = 0; o.epsilon = 1; }
    a.t[k] = MakeTable(tables[t], o);
  }
  for (uint32_t f = 0; f < feature_count; ++f) {
    a.grad[f] = features[f].gradients;
    a.grad_rows[f] = features[f].pooling == EPS_HIP_POOL_SEQUENCE ? features[f].occurrences : features[f].bags;
  }
  if (!reduce) {
    // Vector classes: hot rows (sliced) first, then the other rows per class.
    VecArgs va{};
    for (uint32_t k = 0; k < table_count; ++k) va.t[k] = a.t[k];
    for (uint32_t f = 0; f < feature_count; ++f) {
      va.grad[f] = a.grad[f];
      va.grad_rows[f] = a.grad_rows[f];
    }
    va.tables = table_count;
    va.features = feature_count;
    va.n = a.n;
    va.keys = a.keys;
    va.rs = a.rs;
    va.hot = reinterpret_cast<const HotEntry*>(ws + L.long_list);
    va.hot_capacity = uint32_t(L.HotCapacity());
    va.ctrl = a.ctrl;
    va.bounds = bounds;
    va.gs = a.gs;
    va.spin_limit = SpinLimit();
    va.row_bits = plan.row_bits;
    uint64_t table_refs[EPS_HIP_MAX_TABLES] = {};
    for (uint32_t f = 0; f < feature_count; ++f) table_refs[features[f].table] += features[f].occurrences;
    const bool long_rows = *std::max_element(table_refs, table_refs + table_count) >= kOverlapTableRefs;
    uint64_t vector_occurrences = 0;
    for (uint32_t cls = 0; cls + 1 < kClasses; ++cls) vector_occurrences += plan.class_occurrences[cls];
    // Slice width: pushes with very long hot rows (some table with 65,536 or
    // more references) cut each row into 32-column units, so one row's chain
    // data spreads over several CUs (4 x 8.4 M references: 16-column units
    // 13.8 ms a step, 32-column units, each a whole line per reference, 12.8);
    // small pushes of that kind, whose time is their hottest row's chain and
    // whose gradient rows stay in the caches, take 16-column units, so each
    // chunk moves half the bytes through its producers (65,536 pairs on one
    // table: 100.6 -> 97.0 us an update; a ragged 8-table push of 525,000
    // references lost with them, 270 -> 295 us, and with 256-reference chunks
    // it still did, 264 -> 296 us, as did 4 x 8.4 M references, 9.9 -> 10.8 ms
    // a step); otherwise 64-column units,
    // whose fewer and fuller units a block's producers stage with less
    // bookkeeping per column (26 tables of ~43,000 references: 47 -> 41 us a
    // push).
    const uint32_t slice =
        !long_rows ? kWideSlice : (vector_occurrences < kFinePushRefs ? kFineSlice : kNarrowSlice);
    // Units per hot row: the widest vector table's slices, rounded up to a
    // power of two (units past a row's dimension are skipped in the kernel).
    uint32_t slices = 1;
    for (uint32_t t = 0; t < table_count; ++t)
      if (DimClass(tables[t].dim) < kClasses - 1)
        slices = std::max(slices, (tables[t].dim + slice - 1) / slice);
    va.slice_bits = 0;
    while ((1u << va.slice_bits) < slices) ++va.slice_bits;
    // A hot row takes more than kLongRefs references of its own table, so no
    // table adds more hot rows than its references allow; a push with no such
    // table (a few hundred pairs) launches no hot-row kernel and no events.
    uint64_t hot_rows = 0;
    for (uint32_t t = 0; t < table_count; ++t)
      if (DimClass(tables[t].dim) < kClasses - 1) hot_rows += table_refs[t] / (kLongRefs + 1);
    const uint64_t hot_units = hot_rows << va.slice_bits;
    overlap = hot_units != 0 && !(phases & kOneStream) && t_hot_row_overlap;
    if (phases & kPrimary) {
      // Grids are multiples of kXcds (the kernels split their work by XCD).
      auto xcd_grid = [](uint64_t b) { return (b + kXcds - 1) / kXcds * kXcds; };
      // The hot-row kernel and the row runs side by side on two streams,
      // joined before the checked apply: the longer of the two stays on this
      // stream and the other goes to the side stream, so this stream waits
      // for no event while the longer part runs.  The hot rows are the longer
      // part when some table takes 65,536 or more references (its hottest
      // rows' chains outlast the row runs: 65,536 pairs on one table, hot rows
      // 80 us against row runs 49 us); otherwise the row runs are.  Both
      // sides make the guard decision themselves, from the same snapshot, so
      // they decide the same.
      const bool rows_beside = overlap && long_rows;
      const uint64_t hot_blocks =
          hot_units ? xcd_grid(std::min<uint64_t>(hot_units, long_rows ? kHotGrid : kWideHotGrid)) : 0;
      if (overlap) {
        EPS_HIP_TRY(ThreadOverlap(&ov));
        EPS_HIP_TRY(Check(hipEventRecord(ov->fork, s), "update fork"));
        // With the rows beside, the hot rows (the longer part) go out on this
        // stream before the side stream's wait is set up (the wait on a
        // pending event takes ~14 us of host time): they use no class fields
        // of `va`, and they decide from the same snapshot as the rows.
        if (hot_units && rows_beside) {
          va.role = role;
          EPS_HIP_TRY(LaunchVectorUpdate(0, slice, unsigned(hot_blocks), va, s));
        }
        EPS_HIP_TRY(Check(hipStreamWaitEvent(ov->side, ov->fork, 0), "update fork wait"));
      }
      // The side stream's last kernel records the join as it completes.
      bool joined = false;
      if (hot_units && !rows_beside) {
        va.role = role;
        EPS_HIP_TRY(LaunchVectorUpdate(0, slice, unsigned(hot_blocks), va, overlap ? ov->side : s,
                                       overlap ? ov->join : nullptr));
        joined = overlap;
        if (!overlap) role = kFollow;  // one stream: the hot rows first, deciding; the row kernels follow
      }
      const hipStream_t rs = rows_beside ? ov->side : s;
      // The row runs: one launch per present vector class, or one launch
      // for all of them when there are several.
      uint32_t present = 0;
      uint64_t total_blocks = 0;
      for (uint32_t cls = 0; cls + 1 < kClasses; ++cls) {
        va.class_block[cls] = uint32_t(total_blocks);
        va.class_grid[cls] = 0;
        if (!plan.class_occurrences[cls]) continue;
        const uint64_t blocks = xcd_grid(std::min<uint64_t>(
            std::max<uint64_t>(1, (plan.class_occurrences[cls] + RunPositions(cls + 2) - 1) /
                                      RunPositions(cls + 2)),
            kVectorGrid));
        va.class_grid[cls] = uint32_t(blocks);
        total_blocks += blocks;
        ++present;
      }
      va.class_block[kClasses - 1] = uint32_t(total_blocks);
      va.class_grid[kClasses - 1] = 0;
      // With the rows beside, their launch is the side stream's last (one
      // launch at most: several classes share one).
      const hipEvent_t rows_done = rows_beside ? ov->join : nullptr;
      if (present > 1) {
        va.role = role;
        role = kFollow;
        LaunchRecording(RowRunClassesKernel, dim3(unsigned(total_blocks)), dim3(kBlock), rs, rows_done, va);
        EPS_HIP_LAUNCHED("row update (all classes)");
        joined |= rows_beside;
      } else {
        for (uint32_t cls = 0; cls + 1 < kClasses; ++cls) {
          if (!va.class_grid[cls]) continue;
          va.cls = cls;
          va.role = role;
          role = kFollow;
          EPS_HIP_TRY(LaunchVectorUpdate(cls, 0, va.class_grid[cls], va, rs, rows_done));
          joined |= rows_beside;
        }
      }
      if (overlap && !joined) EPS_HIP_TRY(Check(hipEventRecord(ov->join, ov->side), "update join"));
    }
  }
  for (uint32_t cls = 0; cls < kClasses; ++cls) {
    if (!plan.class_occurrences[cls]) continue;
    if (!reduce && cls + 1 < kClasses) continue;  // handled above
    a.cls = cls;
    a.cls_end = cls + 1;
    a.log2g = cls + 2;
    a.ppb = PositionsPerBlock(cls);
    const uint64_t vb = (plan.class_occurrences[cls] + a.ppb - 1) / a.ppb;
    a.vblocks = uint32_t(vb);
    auto kernel = cls == 5 ? SortedUpdateKernel<true> : SortedUpdateKernel<false>;
    if (phases & kPrimary) {
      a.role = role;
      role = kFollow;
      hipLaunchKernelGGL(kernel, dim3(a.vblocks), dim3(kBlock), 0, s, a);
      EPS_HIP_LAUNCHED("sorted update");
    }
  }
  if (overlap && (phases & kPrimary)) EPS_HIP_TRY(Check(hipStreamWaitEvent(s, ov->join, 0), "hot-row join wait"));
  // The checked apply (after a validate-only pass) is one launch over every
  // class, one wavefront per row: it usually exits at once, and when it runs
  // it adds each row's references in the same order as the passes above.
  if (!reduce && (phases & kSecond)) {
    a.cls = 0;
    a.cls_end = kClasses;
    a.ppb = PositionsPerBlock(kClasses - 1);
    a.vblocks = uint32_t((plan.occurrences + a.ppb - 1) / a.ppb);
    a.role = kFallback;
    if (a.vblocks) {
      hipLaunchKernelGGL(SortedUpdateKernel<true>, dim3(std::min<uint32_t>(a.vblocks, kSecondGrid)),
                         dim3(kBlock), 0, s, a);
      EPS_HIP_LAUNCHED("sorted update (checked apply)");
    }
  }
  return EPS_HIP_OK;
}

}  // namespace
}  // namespace eps_hip

using namespace eps_hip;

extern "C" {

// Shared validation of the push entry points.
static int PushSetup(const eps_hip_table* tables, const eps_hip_optimizer* optimizers,
                     uint32_t table_count, const eps_hip_push_feature* features,
                     uint32_t feature_count, void* workspace, uint64_t workspace_bytes,
                     void* bounds, PushPlan& plan) {
  EPS_HIP_TRY(PlanPush(tables, table_count, features, feature_count, plan));
  const PushLayout L(plan.occurrences);
  if (!workspace || workspace_bytes < L.total)
    return Fail(EPS_HIP_CAPACITY_EXCEEDED, "push workspace too small");
  if (!optimizers || !bounds) return Fail(EPS_HIP_INVALID_ARGUMENT, "push needs optimizers and bounds");
  for (uint32_t t = 0; t < table_count; ++t) EPS_HIP_TRY(CheckOptimizer(optimizers[t]));
  for (uint32_t f = 0; f < feature_count; ++f) {
    const auto& in = features[f];
    const uint64_t rows = in.pooling == EPS_HIP_POOL_SEQUENCE ? in.occurrences : in.bags;
    if (rows && !in.gradients) return Fail(EPS_HIP_INVALID_ARGUMENT, "null feature gradient");
  }
  return EPS_HIP_OK;
}

int eps_hip_push_begin(const eps_hip_table* tables, const eps_hip_optimizer* optimizers,
                       uint32_t table_count, const eps_hip_push_feature* features,
                       uint32_t feature_count, void* workspace, uint64_t workspace_bytes,
                       void* bounds, void* stream) {
  PushPlan plan;
  EPS_HIP_TRY(PushSetup(tables, optimizers, table_count, features, feature_count, workspace,
                        workspace_bytes, bounds, plan));
  GuardArgs g{};
  uint64_t blocks = 0;
  auto add = [&](const void* p, uint64_t count, SpanKind kind) {
    if (!count) return;
    g.span[g.spans++] = Span{static_cast<const float*>(p), count, uint32_t(blocks), kind, 0};
    blocks += SpanBlocks(count, kind);
  };
  for (uint32_t f = 0; f < feature_count; ++f) {
    const auto& in = features[f];
    const uint64_t rows = in.pooling == EPS_HIP_POOL_SEQUENCE ? in.occurrences : in.bags;
    add(in.gradients, rows * tables[in.table].dim, kGradientSpan);
  }
  // The prepared keys, checked before the update uses them as addresses.
  const PushLayout L(plan.occurrences);
  auto* ws = static_cast<uint8_t*>(workspace);
  g.sorted.keys = reinterpret_cast<const uint32_t*>(ws + (plan.passes % 2 == 1 ? L.keys_b : L.keys_a));
  for (uint32_t k = 0; k < table_count; ++k) g.sorted.table_rows[k] = tables[plan.table_of_key[k]].rows;
  g.sorted.row_bits = plan.row_bits;
  g.sorted.tables = table_count;
  add(nullptr, plan.occurrences, kSortedSpan);
  g.ctrl = static_cast<Control*>(workspace);
  g.bounds = static_cast<const Bounds*>(bounds);
  return LaunchGuard(g, blocks, AsStream(stream));
}

static int PushPhase(const eps_hip_table* tables, const eps_hip_optimizer* optimizers,
                     uint32_t table_count, const eps_hip_push_feature* features,
                     uint32_t feature_count, void* workspace, uint64_t workspace_bytes,
                     void* bounds, void* stream, int phase) {
  PushPlan plan;
  EPS_HIP_TRY(PushSetup(tables, optimizers, table_count, features, feature_count, workspace,
                        workspace_bytes, bounds, plan));
  if (!plan.occurrences) return EPS_HIP_OK;
  const PushLayout L(plan.occurrences);
  return RunSorted(tables, optimizers, table_count, features, feature_count, plan, L,
                   static_cast<uint8_t*>(workspace), false, nullptr, nullptr, 0,
                   static_cast<Bounds*>(bounds), AsStream(stream), phase);
}

int eps_hip_push_apply(const eps_hip_table* tables, const eps_hip_optimizer* optimizers,
                       uint32_t table_count, const eps_hip_push_feature* features,
                       uint32_t feature_count, void* workspace, uint64_t workspace_bytes,
                       void* bounds, void* stream) {
  return PushPhase(tables, optimizers, table_count, features, feature_count, workspace,
                   workspace_bytes, bounds, stream, kPrimary);
}

int eps_hip_push_end(const eps_hip_table* tables, const eps_hip_optimizer* optimizers,
                     uint32_t table_count, const eps_hip_push_feature* features,
                     uint32_t feature_count, void* workspace, uint64_t workspace_bytes,
                     void* bounds, void* stream) {
  return PushPhase(tables, optimizers, table_count, features, feature_count, workspace,
                   workspace_bytes, bounds, stream, kSecond);
}

}  // extern "C"

namespace eps_hip {
int PushOneStream(const eps_hip_table* tables, const eps_hip_optimizer* optimizers, uint32_t table_count,
                  const eps_hip_push_feature* features, uint32_t feature_count, void* workspace,
                  uint64_t workspace_bytes, void* bounds, void* stream) {
  EPS_HIP_TRY(eps_hip_push_begin(tables, optimizers, table_count, features, feature_count,
                                 workspace, workspace_bytes, bounds, stream));
  EPS_HIP_TRY(PushPhase(tables, optimizers, table_count, features, feature_count, workspace,
                        workspace_bytes, bounds, stream, kPrimary | kOneStream));
  return PushPhase(tables, optimizers, table_count, features, feature_count, workspace, workspace_bytes,
                   bounds, stream, kSecond | kOneStream);
}
}  // namespace eps_hip

extern "C" {

int eps_hip_push(const eps_hip_table* tables, const eps_hip_optimizer* optimizers,
                 uint32_t table_count, const eps_hip_push_feature* features,
                 uint32_t feature_count, void* workspace, uint64_t workspace_bytes, void* bounds,
                 void* stream) {
  EPS_HIP_TRY(eps_hip_push_begin(tables, optimizers, table_count, features, feature_count,
                                 workspace, workspace_bytes, bounds, stream));
  EPS_HIP_TRY(eps_hip_push_apply(tables, optimizers, table_count, features, feature_count,
                                 workspace, workspace_bytes, bounds, stream));
  return eps_hip_push_end(tables, optimizers, table_count, features, feature_count, workspace,
                          workspace_bytes, bounds, stream);
}

int eps_hip_reduce(const eps_hip_table* tables, uint32_t table_count,
                   const eps_hip_push_feature* features, uint32_t feature_count,
                   void* workspace, uint64_t workspace_bytes, const uint64_t* occurrence_to_unique,
                   float* values, uint64_t row_stride, void* stream) {
  PushPlan plan;
  EPS_HIP_TRY(PlanPush(tables, table_count, features, feature_count, plan));
  const PushLayout L(plan.occurrences);
  if (!workspace || workspace_bytes < L.total)
    return Fail(EPS_HIP_CAPACITY_EXCEEDED, "push workspace too small");
  if (!occurrence_to_unique || !values) return Fail(EPS_HIP_INVALID_ARGUMENT, "null reduce buffers");
  uint32_t max_dim = 0;
  for (uint32_t t = 0; t < table_count; ++t) max_dim = std::max(max_dim, tables[t].dim);
  if (row_stride < max_dim || (row_stride % 4 && max_dim % 4 == 0 && max_dim <= 256))
    return Fail(EPS_HIP_INVALID_ARGUMENT, "row stride must cover every dimension (multiple of 4)");
  EPS_HIP_TRY(PrepareWithOccurrences(tables, table_count, features, feature_count, workspace, workspace_bytes,
                                     stream));
  if (!plan.occurrences) return EPS_HIP_OK;
  auto* ws = static_cast<uint8_t*>(workspace);
  return RunSorted(tables, nullptr, table_count, features, feature_count, plan, L, ws, true,
                   occurrence_to_unique, values, row_stride, nullptr, AsStream(stream), kPrimary);
}

uint64_t eps_hip_update_workspace_bytes(void) { return sizeof(Control); }

static int RunRows(const eps_hip_table* table, const eps_hip_optimizer* optimizer,
                   const uint64_t* slots, uint64_t rows, const uint64_t* offsets,
                   const uint64_t* sources, const float* scales, const float* src,
                   uint64_t src_values, uint64_t references, void* workspace, void* bounds,
                   void* stream) {
  if (!table || !table->state || table->dim == 0 || table->dim > 65536)
    return Fail(EPS_HIP_INVALID_ARGUMENT, "invalid update table");
  if (!optimizer || !workspace || !bounds) return Fail(EPS_HIP_INVALID_ARGUMENT, "null update argument");
  EPS_HIP_TRY(CheckOptimizer(*optimizer));
  const hipStream_t s = AsStream(stream);
  auto* ctrl = static_cast<Control*>(workspace);
  // The control block starts at zero, except the status history (its last word).
  static_assert(kHistoryWord + 1 == sizeof(Control) / 4, "history is the control block's last word");
  EPS_HIP_TRY(LaunchFill(reinterpret_cast<uint32_t*>(ctrl), 0, kHistoryWord, s));
  if (!rows) return EPS_HIP_OK;
  if (!slots || !src) return Fail(EPS_HIP_INVALID_ARGUMENT, "null update buffers");
  GuardArgs g{};
  uint64_t blocks = 0;
  auto add = [&](const void* p, uint64_t count, SpanKind kind, uint64_t limit) {
    if (!count) return;
    g.span[g.spans++] = Span{static_cast<const float*>(p), count, uint32_t(blocks), kind, limit};
    blocks += SpanBlocks(count);
  };
  add(src, src_values, kGradientSpan, 0);
  if (scales) add(scales, references, kScaleSpan, 0);
  // Caller-provided indices are range-checked before the update, so a bad
  // slot or reference rejects it instead of touching memory out of range.
  add(slots, rows, kIndexSpan, table->rows);
  if (offsets) {
    add(offsets, rows + 1, kIndexSpan, references + 1);
    add(sources, references, kIndexSpan, src_values / table->dim);
  }
  const TableDesc d = MakeTable(*table, *optimizer);
  g.ctrl = ctrl;  // the index checks report to its prepare status
  g.bounds = static_cast<const Bounds*>(bounds);
  EPS_HIP_TRY(LaunchGuard(g, blocks, s));
  RowArgs a{};
  a.t = d;
  a.slots = slots;
  a.offsets = offsets;
  a.sources = sources;
  a.scales = scales;
  a.src = src;
  a.rows = rows;
  a.ctrl = ctrl;
  a.bounds = static_cast<Bounds*>(bounds);
  a.gs = GuardScalars{std::max<uint64_t>(1, offsets ? references : 1), 1};
  const uint32_t cls = DimClass(table->dim);
  const bool generic = cls == 5 || reinterpret_cast<uintptr_t>(src) % 16 != 0;
  a.log2g = generic ? 6 : Log2G(table->dim);
  const uint32_t groups = kBlock >> a.log2g;
  const uint64_t vb = (rows + groups - 1) / groups;
  if (vb > 0xffffffffull) return Fail(EPS_HIP_CAPACITY_EXCEEDED, "too many rows");
  a.vblocks = uint32_t(vb);
  auto kernel = generic ? RowUpdateKernel<true> : RowUpdateKernel<false>;
  a.role = kDecide;
  hipLaunchKernelGGL(kernel, dim3(a.vblocks), dim3(kBlock), 0, s, a);
  EPS_HIP_LAUNCHED("row update");
  a.role = kFallback;
  hipLaunchKernelGGL(kernel, dim3(std::min<uint32_t>(a.vblocks, kFallbackGrid)), dim3(kBlock), 0, s, a);
  EPS_HIP_LAUNCHED("row update (checked apply)");
  return EPS_HIP_OK;
}

int eps_hip_adam_rows(const eps_hip_table* table, const eps_hip_optimizer* optimizer,
                      const uint64_t* slots, const float* gradients, uint64_t rows,
                      void* workspace, void* bounds, void* stream) {
  const uint64_t values = table ? rows * table->dim : 0;
  return RunRows(table, optimizer, slots, rows, nullptr, nullptr, nullptr, gradients, values,
                 0, workspace, bounds, stream);
}

int eps_hip_adam_compact(const eps_hip_table* table, const eps_hip_optimizer* optimizer,
                         const uint64_t* slots, uint64_t rows, const uint64_t* row_offsets,
                         const uint64_t* source_rows, const float* scales,
                         const float* source_values, uint64_t source_count, uint64_t references,
                         void* workspace, void* bounds, void* stream) {
  if (rows && (!row_offsets || (references && (!source_rows || !scales))))
    return Fail(EPS_HIP_INVALID_ARGUMENT, "null compact buffers");
  const uint64_t values = table ? source_count * table->dim : 0;
  return RunRows(table, optimizer, slots, rows, row_offsets, source_rows, scales, source_values,
                 values, references, workspace, bounds, stream);
}

uint32_t* eps_hip_status_word(void* workspace) {
  return workspace ? &static_cast<Control*>(workspace)->status : nullptr;
}

uint32_t* eps_hip_status_history_word(void* workspace) {
  return workspace ? &static_cast<Control*>(workspace)->history : nullptr;
}

int eps_hip_set_hot_row_overlap(int enabled) {
  t_hot_row_overlap = enabled != 0;
  return EPS_HIP_OK;
}

int eps_hip_debug_set_spin_limit(uint32_t polls) {
  g_spin_limit.store(polls, std::memory_order_relaxed);
  return EPS_HIP_OK;
}

int eps_hip_read_status(void* workspace, uint32_t* status, void* stream) {
  if (!workspace || !status) return Fail(EPS_HIP_INVALID_ARGUMENT, "null status arguments");
  EPS_HIP_TRY(Check(hipStreamSynchronize(AsStream(stream)), "hipStreamSynchronize"));
  EPS_HIP_TRY(Check(hipMemcpy(status, &static_cast<Control*>(workspace)->status, 4,
                              hipMemcpyDeviceToHost), "status copy"));
  return EPS_HIP_OK;
}

}  // extern "C"
