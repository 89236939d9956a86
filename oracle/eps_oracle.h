/*
 * eps_oracle.h -- CPU restatement of the reference parameter-shard path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker for the HIP
 * implementation: only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it.  The product path never calls it.
 *
 * Everything here follows the reference algorithms and floating-point
 * operation order exactly (compiled with -ffp-contract=off, no -march, so
 * float arithmetic is IEEE binary32 on SSE2).  Citations are to the reference
 * repository (Zhang-Xin-Duke/distributed-recommendation-model-training-system).
 *
 * Parity pins (each function is checked by tests/test_oracle_*.py against the
 * reference's own known-answer tests, closed forms, brute force, and -- where
 * oracle/_ref is built -- against the compiled reference sources):
 *   init / ensure      : tests/core_tests.cpp:142-154 (topology independence),
 *                        reference build (bit-exact weights)
 *   prepare_feature    : tests/core_tests.cpp:68-75, reference build
 *   reduce_gradients   : tests/core_tests.cpp:76-82, tests/compact_tests.cpp,
 *                        reference build
 *   lazy_adam          : tests/core_tests.cpp:78-82, weight_bounds_tests.cpp:78-86,
 *                        core_tests.cpp:214-222 (atomic reject), reference build
 *   compact build/expand: tests/compact_tests.cpp:13-40, reference build
 *   gather_host / adam_ctx: tests/cuda_tests.cpp:35-139 shapes, reference build
 *   weighted-sum pooling: extension with no reference counterpart; pinned by
 *                        closed form (reduces to sum pooling at unit weights and
 *                        to brute-force float loops otherwise).
 */
#ifndef EPS_ORACLE_H
#define EPS_ORACLE_H
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

/* Status codes: 0 ok, else eps::Error::Code + 1 (include/eps/types.hpp:17-22). */
#define EPS_OR_OK 0
#define EPS_OR_INVALID_ARGUMENT 1
#define EPS_OR_UNAVAILABLE 2
#define EPS_OR_STALE_GENERATION 3
#define EPS_OR_CAPACITY_EXCEEDED 5

/* Pooling modes: include/eps/types.hpp:51 (sum, mean, sequence) + weighted sum. */
#define EPS_OR_SUM 0
#define EPS_OR_MEAN 1
#define EPS_OR_SEQUENCE 2
#define EPS_OR_WEIGHTED_SUM 3

typedef struct eps_or_table_def {
  uint32_t id, dim, shard, shard_count;
  float learning_rate, beta1, beta2, epsilon;
  float initial_beta1_power, initial_beta2_power;
  int32_t bounded;
  float weight_min, weight_max;
  float init_min, init_max;
  uint64_t init_seed;
} eps_or_table_def;

typedef struct eps_or_feature {
  const uint64_t* keys;
  uint64_t key_count;
  const uint64_t* offsets;       /* bag_count + 1 entries */
  const uint64_t* valid_lengths; /* bag_count entries */
  const float* weights;          /* per key; weighted-sum pooling only */
  uint64_t bag_count;
  uint32_t pooling;
  uint32_t feature;
} eps_or_feature;

typedef struct eps_or_store eps_or_store;

const char* eps_or_last_error(void);

/* ---- row store: src/store/shard_store.cpp ---- */
uint64_t eps_or_mix(uint64_t x);
float eps_or_init_weight(const eps_or_table_def* t, uint64_t key, uint32_t d);
eps_or_store* eps_or_create(const eps_or_table_def* t);
void eps_or_destroy(eps_or_store* s);
int64_t eps_or_ensure(eps_or_store* s, uint64_t key);
int64_t eps_or_find(const eps_or_store* s, uint64_t key);
uint64_t eps_or_row_count(const eps_or_store* s);
uint64_t eps_or_key_at(const eps_or_store* s, uint64_t slot);
int eps_or_read(const eps_or_store* s, uint64_t key, float* w, float* m, float* v,
                uint64_t* updates);
int eps_or_import(eps_or_store* s, uint64_t key, const float* w, const float* m,
                  const float* v, uint64_t updates);
int eps_or_overwrite(eps_or_store* s, uint64_t key, const float* w, const float* m,
                     const float* v, uint64_t updates);
int eps_or_read_many(const eps_or_store* s, const uint64_t* keys, uint64_t count,
                     float* packed, uint64_t* updates, uint64_t* keys_out);
void eps_or_powers(const eps_or_store* s, float* beta1_power, float* beta2_power,
                   uint64_t* optimizer_sequence);

/* ---- pull: src/access/batch_access.cpp, src/client/distributed_client.cpp ---- */
int eps_or_prepare_feature(eps_or_store* s, const eps_or_feature* f,
                           uint64_t* unique_slots, uint64_t* unique_count,
                           uint64_t* occurrence_to_unique, float* contribution);
void eps_or_mean_divide(float* values, const uint64_t* valid_lengths, uint64_t bags,
                        uint32_t dim);

/* ---- push: batch_access.cpp ReduceGradients, lazy_adam.cpp ---- */
int eps_or_reduce_gradients(const eps_or_store* s, const eps_or_feature* features,
                            const float* const* gradients, uint32_t feature_count,
                            uint64_t* row_keys, float* row_values, uint64_t* row_count);
float eps_or_lr_t(float learning_rate, float beta1_power, float beta2_power);
int eps_or_validate_lazy_adam(const eps_or_store* s, const uint64_t* keys,
                              const float* gradients, uint64_t rows);
void eps_or_apply_lazy_adam(eps_or_store* s, const uint64_t* keys,
                            const float* gradients, uint64_t rows);
int eps_or_push(eps_or_store* const* stores, uint32_t store_count,
                const eps_or_feature* features, const uint32_t* feature_store,
                const float* const* gradients, uint32_t feature_count);

/* ---- backend semantics: src/cache/host_backend.cpp, compact_gradients.cpp ---- */
int eps_or_adam_rows_ctx(float* weights, float* first, float* second,
                         const float* gradients, uint64_t rows, uint32_t dim,
                         float beta1, float beta2, float epsilon, float learning_rate,
                         float beta1_power, float beta2_power, int32_t bounded,
                         float weight_min, float weight_max);
int eps_or_gather_host(const eps_or_feature* f, uint32_t dim,
                       const uint64_t* occurrence_to_unique, uint64_t unique_count,
                       const float* const* unique_weights, float* out);
uint64_t eps_or_compact_bytes(uint64_t rows, uint64_t source_values, uint64_t references);
int eps_or_validate_compact(uint64_t rows, const uint64_t* row_keys, uint32_t dim,
                            const float* source_values, uint64_t source_value_count,
                            const uint64_t* row_offsets, const uint64_t* source_rows,
                            const float* scales, uint64_t references);
int eps_or_expand_compact(uint64_t rows, const uint64_t* row_keys, uint32_t dim,
                          const float* source_values, uint64_t source_value_count,
                          const uint64_t* row_offsets, const uint64_t* source_rows,
                          const float* scales, uint64_t references, float* out);
int eps_or_build_compact(const eps_or_feature* features, const float* const* gradients,
                         uint32_t feature_count, uint32_t dim, const uint64_t* row_keys,
                         uint64_t rows, float* source_values, uint64_t* source_value_count,
                         uint64_t* row_offsets, uint64_t* source_rows, float* scales,
                         uint64_t* references);

/* ---- snapshot format: src/store/snapshot.cpp ---- */
#define EPS_OR_FNV_OFFSET 14695981039346656037ULL
/* FNV-1a (64-bit) over `size` bytes, continuing from `hash`. */
uint64_t eps_or_fnv1a(uint64_t hash, const void* data, uint64_t size);
/* WriteSnapshot (snapshot.cpp:159-194): format 2, the tables in the order given
 * (the reference writes its hash map's order), each table's rows in its store's
 * key order, every table's partition epoch = epoch.  Writes `path` directly. */
int eps_or_snapshot_write(const char* path, const char* run, uint64_t shard,
                          uint64_t shard_count, uint64_t epoch, eps_or_store* const* stores,
                          uint32_t table_count);
/* ReadSnapshot (snapshot.cpp:221-267) of format 1 or 2 into new stores, tables
 * in file order (the caller destroys them).  run receives the NUL-terminated
 * run ID (run_capacity >= 1025). */
int eps_or_snapshot_read(const char* path, char* run, uint64_t run_capacity, uint64_t* shard,
                         uint64_t* shard_count, uint64_t* epoch, uint32_t* version,
                         eps_or_store** stores, uint32_t capacity, uint32_t* table_count,
                         uint64_t* checksum);

#ifdef __cplusplus
}
#endif
#endif
