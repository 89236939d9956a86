/*
 * eps_hip.h -- C ABI of the MI355X (gfx950) parameter-shard embedding path.
 *
 * This is the kernel layer below the C++ backend (eps::HipCacheBackend): it
 * replaces the seven CUDA kernels and their launch helpers in the reference's
 * src/cuda/cache_backend.cu, and adds the device-side dedup/aggregation that the
 * reference performs on the host.  Every entry point:
 *   - returns 0 on success, else eps::Error::Code + 1 (include/eps/types.hpp:17-22,
 *     the same mapping the reference C runtime uses, adapters/entropy/runtime_c.cpp:21-30),
 *     with a message from eps_hip_last_error();
 *   - takes caller-owned device buffers and an explicit hipStream_t (as void*);
 *   - enqueues work on that stream and returns without synchronising, except
 *     eps_hip_read_status which waits for the stream;
 *   - never allocates device memory: scratch space is a caller-provided
 *     workspace sized by the matching *_workspace_bytes query (or, for
 *     eps_hip_push_static, a static array of the library).
 * Data-dependent outcomes (out-of-range row slots, non-finite gradients,
 * optimizer overflow) are reported in a device status word of the workspace,
 * read with eps_hip_read_status after the stream has drained.
 *
 * Device table layout: one allocation per table, `rows` slots, each slot a
 * contiguous array-of-structures row [w(dim) | m(dim) | v(dim)] of fp32
 * (reference layout: src/store/shard_store.cpp:21-29; device
 * src/cuda/cache_backend.cu:101).  `state` must be 16-byte aligned.
 */
#ifndef EPS_HIP_H
#define EPS_HIP_H
#include <stddef.h>
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

#define EPS_HIP_ABI_VERSION 1

/* Status codes (eps::Error::Code + 1). */
#define EPS_HIP_OK 0
#define EPS_HIP_INVALID_ARGUMENT 1
#define EPS_HIP_UNAVAILABLE 2
#define EPS_HIP_STALE_GENERATION 3
#define EPS_HIP_RETIRED_REQUEST 4
#define EPS_HIP_CAPACITY_EXCEEDED 5
#define EPS_HIP_RUN_FAILED 6

/* Pooling modes: eps::Pooling (include/eps/types.hpp:51) plus weighted sum. */
#define EPS_HIP_POOL_SUM 0
#define EPS_HIP_POOL_MEAN 1
#define EPS_HIP_POOL_SEQUENCE 2
#define EPS_HIP_POOL_WEIGHTED_SUM 3

/* Bits of the device status word (0 = the update was applied). */
#define EPS_HIP_STATUS_BAD_INDEX 0x1u        /* a row slot >= table rows */
#define EPS_HIP_STATUS_NONFINITE_GRAD 0x2u   /* batch_access.cpp:23-24 */
#define EPS_HIP_STATUS_REDUCE_OVERFLOW 0x4u  /* batch_access.cpp:95 */
#define EPS_HIP_STATUS_ADAM_OVERFLOW 0x8u    /* lazy_adam.cpp:19-20 */
#define EPS_HIP_STATUS_REJECTED 0x10u        /* nothing was written */
#define EPS_HIP_STATUS_STALLED 0x20u         /* internal: a hot-row hand-over timed out */
#define EPS_HIP_STATUS_BAD_SCALE 0x40u       /* a non-finite reference scale or per-id weight,
                                                or a negative compact scale
                                                (compact_gradients.cpp:21) */
#define EPS_HIP_STATUS_CHECKED_PATH 0x100u   /* info: the two-pass path ran */

/* Per-launch limits (descriptors travel as kernel arguments). */
#define EPS_HIP_MAX_FEATURES 32
#define EPS_HIP_MAX_TABLES 32
#define EPS_HIP_MAX_GATHER_PARTS 32

typedef struct eps_hip_table {
  float* state;       /* rows * 3 * dim floats */
  uint64_t rows;      /* slot capacity */
  uint32_t dim;
  uint32_t id;        /* eps::TableId; initializer input */
} eps_hip_table;

/* Optimizer context of one table for one update: OptimizerConfig
 * (include/eps/types.hpp:76-86) with the UpdateContext powers (:181-189). */
typedef struct eps_hip_optimizer {
  float learning_rate, beta1, beta2, epsilon;
  float beta1_power, beta2_power;
  int32_t bounded;
  float weight_min, weight_max;
} eps_hip_optimizer;

/* One pooled-gather part (one feature).  Replaces GatherKernel + NormalizeMean
 * (src/cuda/cache_backend.cu:81-94,134-139) as laid out by PrepareGather
 * (:251-308). */
typedef struct eps_hip_gather_part {
  const float* source;            /* table state (stride 3*dim) or unique vectors (stride dim) */
  const uint64_t* indices;        /* per occurrence; UINT64_MAX = not here (skipped);
                                     NULL allowed for a pooled part of empty bags */
  const uint64_t* remap;          /* optional: slot = remap[indices[i]] (unique -> slot) */
  const uint64_t* offsets;        /* bag_count + 1 (pooled modes) */
  const uint64_t* valid_lengths;  /* mean only: divide by it when non-NULL (client mean) */
  const float* weights;           /* per occurrence, weighted sum only */
  float* output;                  /* rows * dim, row-major */
  uint64_t stride;                /* floats between slots */
  uint64_t rows;                  /* bags, or occurrences for sequence */
  uint64_t source_rows;           /* slots >= this are rejected (status bit) */
  uint64_t remap_count;           /* entries of remap */
  uint32_t dim;
  uint32_t pooling;
} eps_hip_gather_part;

/* One feature of a device-side push: the lookup's layout plus its gradient.
 * Mirrors FeatureInput (include/eps/types.hpp:100-109) + TensorBlock (:111-115). */
typedef struct eps_hip_push_feature {
  const uint64_t* indices;        /* per occurrence slot; UINT64_MAX = not here */
  const uint64_t* offsets;        /* bags + 1 */
  const uint64_t* valid_lengths;  /* bags (mean scale 1.0f/len) */
  const float* weights;           /* per occurrence (weighted sum) */
  const float* gradients;         /* (bags, or occurrences for sequence) * dim */
  uint64_t occurrences;
  uint64_t bags;
  uint32_t table;                 /* index into the call's table array */
  uint32_t pooling;
} eps_hip_push_feature;

int eps_hip_abi_version(void);
const char* eps_hip_last_error(void);
/* Verifies the device is a gfx950 (MI355X) and makes it current. */
int eps_hip_device_check(int device);

/* ---- optimizer-state bounds domain (sound single-pass overflow guard) ---- */
/* A small device buffer holding running upper bounds of |w|, |m| and v over all
 * state written through this library; the fused update uses it to prove that no
 * element can overflow before it writes (the guard is described in csrc/adam.hip). */
uint64_t eps_hip_bounds_bytes(void);
int eps_hip_bounds_reset(void* bounds, void* stream);

/* ---- row state ---- */
/* Reference initializer for slots [first, first+count): key = key_base +
 * slot * key_stride; w = ShardStore::Ensure's SplitMix64 uniform
 * (src/store/shard_store.cpp:104-112), m = v = 0.  Replaces first-touch init. */
int eps_hip_init_rows(const eps_hip_table* table, uint64_t first_slot, uint64_t count,
                      uint64_t key_base, uint64_t key_stride, uint64_t seed,
                      float init_min, float init_max, int32_t bounded, float weight_min,
                      float weight_max, void* bounds, void* stream);
/* Cache admission: packed rows [w|m|v] -> slots.  Replaces ScatterState
 * (src/cuda/cache_backend.cu:69-74) as used by Load (:390-462).  `packed` may be
 * device memory or pinned host memory (read over the host link directly). */
int eps_hip_scatter_rows(const eps_hip_table* table, const uint64_t* slots,
                         const float* packed, uint64_t count, void* bounds, void* stream);
/* Writeback: slots -> packed rows.  Replaces ReadStateKernel (:75-80) as used by
 * ReadBack (:540-585).  `packed` may be pinned host memory. */
int eps_hip_gather_rows(const eps_hip_table* table, const uint64_t* slots, float* packed,
                        uint64_t count, void* stream);

/* Row moves of up to EPS_HIP_MAX_TABLES tables in one launch: the tier moves
 * of a step (Load's ScatterState and ReadBack's ReadStateKernel,
 * src/cuda/cache_backend.cu:69-80,390-585, once per table there).  With
 * write_back 0, batch b's packed rows [w|m|v] go to its slots (bounds updated,
 * as eps_hip_scatter_rows); with write_back 1, its slots' rows go to `packed`
 * (as eps_hip_gather_rows).  `packed` may be device or pinned host memory. */
typedef struct eps_hip_row_batch {
  float* state;          /* the table's state (16-byte aligned) */
  const uint64_t* slots; /* count slots */
  float* packed;         /* count x 3 x dim floats */
  uint64_t count;
  uint32_t dim;
  uint32_t reserved;
} eps_hip_row_batch;
int eps_hip_move_rows(const eps_hip_row_batch* batches, uint32_t count, int32_t write_back,
                      void* bounds, void* stream);

/* ---- device key -> slot index of a table ---- */
/* The reference keeps a host hash map per table (CudaCacheBackend's
 * Table::rows, src/cuda/cache_backend.cu:193-198) and looks every key
 * occurrence up in it on the host before a gather (:279-291).  This index is
 * an open-addressing hash table in device memory (16 bytes per bucket,
 * `capacity` a power of two, at most half full for short probes) that
 * admissions insert into and evictions remove from, so occurrences resolve on
 * the device.  Keys of one insert or remove call must be distinct; a key must
 * not be inserted twice.  Failures (a full index, removing a key that is not
 * there) set EPS_HIP_STATUS_BAD_INDEX in `status` (device u32, may be NULL).
 * A removed key leaves a marker bucket that inserts reuse but nothing empties,
 * so an owner that removes keys rebuilds the index (clear, then insert the
 * live keys) after removals to a quarter of `capacity`; HipCacheBackend does. */
uint64_t eps_hip_index_bytes(uint64_t capacity);
int eps_hip_index_clear(void* index, uint64_t capacity, void* stream);
int eps_hip_index_insert(void* index, uint64_t capacity, const uint64_t* keys, const uint64_t* slots,
                         uint64_t count, uint32_t* status, void* stream);
int eps_hip_index_remove(void* index, uint64_t capacity, const uint64_t* keys, uint64_t count,
                         uint32_t* status, void* stream);
/* Slots of n key occurrences (the per-occurrence part of PrepareGather,
 * :279-291).  With `occurrence_to_unique` (the lookup's AgentWork map): a
 * UINT64_MAX entry stays a hole; otherwise occurrence i must name its unique
 * row (keys[i] == unique_keys[occurrence_to_unique[i]]) and resolves through
 * `index` to that row's slot, or, with no index, to the unique index itself
 * (rows carried with the request).  Without a map, keys absent from the index
 * become holes.  Any mismatch sets BAD_INDEX in `status` (the reference's
 * "invalid occurrence map") and resolves to a hole. */
int eps_hip_resolve(const void* index, uint64_t capacity, const uint64_t* keys,
                    const uint64_t* occurrence_to_unique, const uint64_t* unique_keys,
                    uint64_t unique_count, uint64_t n, uint64_t* slots, uint32_t* status,
                    void* stream);

/* ---- pull ---- */
/* Pooled gather of up to EPS_HIP_MAX_GATHER_PARTS features in one launch.
 * Replaces LaunchGather/GatherKernel (:309-320,81-94) and fuses NormalizeMean
 * (:134-139) when valid_lengths is given.  `status` (device u32, may be NULL)
 * receives EPS_HIP_STATUS_BAD_INDEX for out-of-range slots (skipped). */
int eps_hip_gather(const eps_hip_gather_part* parts, uint32_t count, uint32_t* status,
                   void* stream);
/* Elementwise output[i] += source[i] (or output[positions[i/dim]*dim + i%dim]).
 * Replaces AddContribution (:126-133). */
int eps_hip_add_contribution(float* output, const float* source, const uint64_t* positions,
                             uint64_t values, uint32_t dim, void* stream);

/* In-place mean of assembled pooled sums: output[r*dim + d] /= (float)lengths[r]
 * where lengths[r] != 0.  Replaces NormalizeMean (:134-139) as used by
 * AssembleFeatures (:686-692). */
int eps_hip_normalize_mean(float* output, const uint64_t* lengths, uint64_t rows, uint32_t dim,
                           void* stream);

/* ---- push: device dedup + duplicate-id aggregation + fused sparse Adam ---- */
/* Workspace for up to `occurrences` total occurrences over the call's features. */
uint64_t eps_hip_push_workspace_bytes(uint64_t occurrences);
/* Lookup-time preparation of a push (the device counterpart of PrepareFeature's
 * dedup, batch_access.cpp:32-36, and of the occurrence maps in the lookup ticket):
 * stable radix sort of occurrences by (table, slot).  Uses features' indices,
 * offsets, valid_lengths and weights; not their gradients. */
int eps_hip_prepare(const eps_hip_table* tables, uint32_t table_count,
                    const eps_hip_push_feature* features, uint32_t feature_count,
                    void* workspace, uint64_t workspace_bytes, void* stream);
/* Push of a prepared workspace: ReduceGradients (batch_access.cpp:54-97) +
 * ValidateLazyAdam/ApplyLazyAdam (lazy_adam.cpp:7-42) per table, in one fused
 * read-modify-write of each unique row, all-or-nothing over the call.  Uses the
 * features' gradients (same features, same order as eps_hip_prepare). */
int eps_hip_push(const eps_hip_table* tables, const eps_hip_optimizer* optimizers,
                 uint32_t table_count, const eps_hip_push_feature* features,
                 uint32_t feature_count, void* workspace, uint64_t workspace_bytes,
                 void* bounds, void* stream);
/* The three stream-ordered phases of eps_hip_push, for callers that overlap or
 * time them: begin = gradient scan + overflow guard decision; apply = the fused
 * aggregation + Adam pass (validate-only when the guard cannot prove safety);
 * end = the second (apply) pass of that checked case, a no-op otherwise. */
int eps_hip_push_begin(const eps_hip_table* tables, const eps_hip_optimizer* optimizers,
                       uint32_t table_count, const eps_hip_push_feature* features,
                       uint32_t feature_count, void* workspace, uint64_t workspace_bytes,
                       void* bounds, void* stream);
int eps_hip_push_apply(const eps_hip_table* tables, const eps_hip_optimizer* optimizers,
                       uint32_t table_count, const eps_hip_push_feature* features,
                       uint32_t feature_count, void* workspace, uint64_t workspace_bytes,
                       void* bounds, void* stream);
int eps_hip_push_end(const eps_hip_table* tables, const eps_hip_optimizer* optimizers,
                     uint32_t table_count, const eps_hip_push_feature* features,
                     uint32_t feature_count, void* workspace, uint64_t workspace_bytes,
                     void* bounds, void* stream);
/* Unique rows of the features in first-occurrence order (PrepareFeature /
 * ReduceGradients row order): unique_slots[u], unique_tables[u],
 * occurrence_to_unique[i] (UINT64_MAX for holes), and the count (device u64).
 * Prepares the workspace itself, keeping each sorted position's occurrence
 * index (which eps_hip_prepare leaves out); the workspace then also serves
 * eps_hip_push. */
int eps_hip_unique(const eps_hip_table* tables, uint32_t table_count,
                   const eps_hip_push_feature* features, uint32_t feature_count,
                   void* workspace, uint64_t workspace_bytes, uint64_t* unique_slots,
                   uint32_t* unique_tables, uint64_t* occurrence_to_unique,
                   uint64_t* unique_count, void* stream);
/* ReduceGradients values with eps_hip_unique's occurrence map: row u written
 * at values + u * row_stride (first-occurrence order).  Prepares the workspace
 * itself, as eps_hip_unique does. */
int eps_hip_reduce(const eps_hip_table* tables, uint32_t table_count,
                   const eps_hip_push_feature* features, uint32_t feature_count,
                   void* workspace, uint64_t workspace_bytes,
                   const uint64_t* occurrence_to_unique, float* values,
                   uint64_t row_stride, void* stream);

/* A device push that allocates nothing.  No counterpart in the reference: it
 * is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops).  Same as eps_hip_prepare + eps_hip_push on
 * the same arguments, with the push workspace in a static device array of this
 * library (about 12 MB per GPU, held from the library's load until the process
 * ends) instead of a caller's buffer; pushes of more than
 * EPS_HIP_STATIC_MAX_OCCURRENCES occurrences are refused with
 * EPS_HIP_CAPACITY_EXCEEDED before anything is enqueued.  `status` (device
 * memory, 2 u32, may be NULL) receives the push's status word and the array's
 * status history (the failure bits of every static push since the last call
 * that passed `status`, which then clears it) once the push has run.  Every
 * kernel runs on `stream`, the hot-row kernel before the row kernels (no side
 * stream or event), so once a device's first call has looked up the array's
 * address a call can be captured in a graph.  Every call on one GPU shares
 * that GPU's array: calls that overlap on one GPU race. */
#define EPS_HIP_STATIC_MAX_OCCURRENCES 262144u
int eps_hip_push_static(const eps_hip_table* tables, const eps_hip_optimizer* optimizers,
                        uint32_t table_count, const eps_hip_push_feature* features,
                        uint32_t feature_count, void* bounds, uint32_t* status, void* stream);

/* ---- backend updates with host-built layouts ---- */
uint64_t eps_hip_update_workspace_bytes(void);
/* ApplyHost: unique rows with reduced gradients.  Replaces ApplyPrepared's two
 * AdamKernel launches (src/cuda/cache_backend.cu:95-114,334-350). */
int eps_hip_adam_rows(const eps_hip_table* table, const eps_hip_optimizer* optimizer,
                      const uint64_t* slots, const float* gradients, uint64_t rows,
                      void* workspace, void* bounds, void* stream);
/* ApplyCompact: CSR references (CompactGradients, include/eps/types.hpp:197-206)
 * reduced and applied in one pass.  Replaces ReduceFeatureGradients + the
 * AdamKernel pair (:115-125,514-538). */
int eps_hip_adam_compact(const eps_hip_table* table, const eps_hip_optimizer* optimizer,
                         const uint64_t* slots, uint64_t rows, const uint64_t* row_offsets,
                         const uint64_t* source_rows, const float* scales,
                         const float* source_values, uint64_t source_count,
                         uint64_t references, void* workspace, void* bounds, void* stream);

/* ---- status ---- */
/* Device address of the status word inside a push or update workspace.  A
 * call's status is complete once its last enqueued kernel has run (a push:
 * after eps_hip_push_end).  Any bit of 0x7f means the call failed; with any
 * failure bit but EPS_HIP_STATUS_STALLED, nothing was written.  A stall (a
 * hot-row hand-over that exceeded its spin limit, which no correct run
 * reaches) writes none of the stalled work units' rows; rows of other work
 * units of the same push may have been written (the hot-row kernel runs beside
 * the row kernels, except in eps_hip_push_static), so the tables are to be
 * restored, e.g. from a snapshot; eps::HipCacheBackend stops after one.  A
 * bad-index bit from a push whose prepared keys were in range (a damaged
 * reference word) likewise leaves the rows that reference fed unwritten and
 * others written. */
uint32_t* eps_hip_status_word(void* workspace);
/* Device address of the workspace's status history: the OR of the failure
 * bits of every push or update run in it since it was zeroed (a workspace
 * must be zero-filled once when it is allocated; the calls themselves never
 * clear this word).  For callers that enqueue many pushes without reading
 * each status; clear it with eps_hip_fill_u32. */
uint32_t* eps_hip_status_history_word(void* workspace);
/* Waits for `stream` and copies the workspace status word to *status. */
int eps_hip_read_status(void* workspace, uint32_t* status, void* stream);
/* Fills count u32 words with value (a kernel, safe under graph capture). */
int eps_hip_fill_u32(uint32_t* target, uint32_t value, uint64_t count, void* stream);

/* Where this thread's pushes run the hot-row kernel (rows with more than 128
 * references).  Enabled (the default): beside the row kernels on two streams,
 * the push's stream and a side stream the library creates per thread and
 * device, forked after the gradient scan and joined before the checked apply;
 * the side stream takes the row kernels when some table of the push has
 * 65,536 or more references (its hot rows outlast them), else the hot-row
 * kernel.  Disabled: both on the push's stream, hot rows first (as
 * eps_hip_push_static does).  A push whose tables each take 128 or fewer
 * references has no hot rows and uses no side stream.  No counterpart in the
 * reference.  The side stream pays off when it has a hardware queue of its
 * own: HIP maps a process's streams onto GPU_MAX_HW_QUEUES queues (4 by
 * default) round robin, so a caller that keeps more streams busy than there
 * are queues (e.g. a pipeline with cache-tier copy streams) should disable
 * it.  Per calling thread; returns EPS_HIP_OK. */
int eps_hip_set_hot_row_overlap(int enabled);

/* Test hook: polls of an LDS hand-over wait of the hot-row kernel before it
 * gives up (default 4194304; process-wide).  0 makes every such wait give up
 * at once, so tests can drive the stall path from the host. */
int eps_hip_debug_set_spin_limit(uint32_t polls);

#ifdef __cplusplus
}
#endif
#endif
