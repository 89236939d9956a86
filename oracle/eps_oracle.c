/*
 * eps_oracle.c -- CPU restatement of the reference parameter-shard path.
 *
 * TEST INFRASTRUCTURE ONLY (see eps_oracle.h): the checker for the HIP path and
 * the timed CPU baseline.  Never linked into the product library.
 *
 * Build: gcc -O2 -ffp-contract=off -fPIC -shared (no -march, no fast-math), so
 * every float operation below is one correctly rounded IEEE binary32 operation
 * in the order written, as in the reference Release build.
 */
#include "eps_oracle.h"

#include <float.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static __thread char g_error[256];
static int fail(int code, const char* message) {
  snprintf(g_error, sizeof g_error, "%s", message);
  return code;
}
const char* eps_or_last_error(void) { return g_error; }

/* ------------------------------------------------------------------------ */
/* u64 -> u64 open-addressing map (stands in for std::unordered_map).        */
typedef struct omap {
  uint64_t* keys;
  uint64_t* vals;
  uint8_t* used;
  uint64_t cap, size;
} omap;

static uint64_t hash64(uint64_t x) {
  x ^= x >> 33; x *= 0xff51afd7ed558ccdULL; x ^= x >> 33;
  x *= 0xc4ceb9fe1a85ec53ULL; x ^= x >> 33;
  return x;
}
static void omap_init(omap* m, uint64_t expected) {
  uint64_t cap = 16;
  while (cap < expected * 2 + 16) cap <<= 1;
  m->keys = (uint64_t*)malloc(cap * sizeof(uint64_t));
  m->vals = (uint64_t*)malloc(cap * sizeof(uint64_t));
  m->used = (uint8_t*)calloc(cap, 1);
  m->cap = cap; m->size = 0;
}
static void omap_free(omap* m) { free(m->keys); free(m->vals); free(m->used); }
static int64_t omap_find(const omap* m, uint64_t key) {
  uint64_t i = hash64(key) & (m->cap - 1);
  while (m->used[i]) {
    if (m->keys[i] == key) return (int64_t)m->vals[i];
    i = (i + 1) & (m->cap - 1);
  }
  return -1;
}
static void omap_grow(omap* m);
/* Returns the existing value, or inserts `value` and returns -1. */
static int64_t omap_try_emplace(omap* m, uint64_t key, uint64_t value) {
  if ((m->size + 1) * 2 > m->cap) omap_grow(m);
  uint64_t i = hash64(key) & (m->cap - 1);
  while (m->used[i]) {
    if (m->keys[i] == key) return (int64_t)m->vals[i];
    i = (i + 1) & (m->cap - 1);
  }
  m->used[i] = 1; m->keys[i] = key; m->vals[i] = value; ++m->size;
  return -1;
}
static void omap_grow(omap* m) {
  omap n; omap_init(&n, m->cap);
  for (uint64_t i = 0; i < m->cap; ++i)
    if (m->used[i]) omap_try_emplace(&n, m->keys[i], m->vals[i]);
  omap_free(m); *m = n;
}

/* ------------------------------------------------------------------------ */
/* Row store.  Layout per row [w(dim) | m(dim) | v(dim)] + u64 update counter,
 * slots assigned in first-touch order: src/store/shard_store.cpp:21-29,76-115. */
struct eps_or_store {
  eps_or_table_def def;
  float beta1_power, beta2_power;
  uint64_t optimizer_sequence;
  omap index;
  uint64_t* keys;
  float* values;
  uint64_t* updates;
  uint64_t rows, cap;
};

/* SplitMix64 finaliser: src/store/shard_store.cpp:13-18. */
uint64_t eps_or_mix(uint64_t x) {
  x += 0x9e3779b97f4a7c15ULL;
  x = (x ^ (x >> 30)) * 0xbf58476d1ce4e5b9ULL;
  x = (x ^ (x >> 27)) * 0x94d049bb133111ebULL;
  return x ^ (x >> 31);
}

/* BoundWeight: src/common/optimizer_bounds.hpp:14-18 (std::clamp(v, lo, hi)). */
static float bound_weight(float value, int32_t bounded, float lo, float hi) {
  if (!bounded) return value;
  return value < lo ? lo : (hi < value ? hi : value);
}

/* Initializer: src/store/shard_store.cpp:104-112.  u in [0,1) from the top 53
 * bits, lerp in double, one rounding to float, then the weight clamp. */
float eps_or_init_weight(const eps_or_table_def* t, uint64_t key, uint32_t d) {
  const uint64_t bits = eps_or_mix(key ^ eps_or_mix(t->init_seed) ^
                                   eps_or_mix((uint64_t)t->id) ^ eps_or_mix((uint64_t)d));
  const double u = (double)(bits >> 11) * 0x1.0p-53;
  const float w = (float)((1 - u) * (double)t->init_min + u * (double)t->init_max);
  return bound_weight(w, t->bounded, t->weight_min, t->weight_max);
}

eps_or_store* eps_or_create(const eps_or_table_def* t) {
  /* Validation as in ShardStore::Create, shard_store.cpp:37-52. */
  if (t->dim == 0 || t->dim > 65536 || t->shard_count == 0 || t->shard >= t->shard_count) {
    fail(EPS_OR_INVALID_ARGUMENT, "invalid table definition");
    return NULL;
  }
  if (t->bounded && !(isfinite(t->weight_min) && isfinite(t->weight_max) &&
                      t->weight_min <= t->weight_max)) {
    fail(EPS_OR_INVALID_ARGUMENT, "invalid optimizer weight bounds");
    return NULL;
  }
  eps_or_store* s = (eps_or_store*)calloc(1, sizeof *s);
  s->def = *t;
  s->beta1_power = t->initial_beta1_power;
  s->beta2_power = t->initial_beta2_power;
  omap_init(&s->index, 1024);
  s->cap = 1024;
  s->keys = (uint64_t*)malloc(s->cap * sizeof(uint64_t));
  s->values = (float*)malloc(s->cap * (uint64_t)t->dim * 3 * sizeof(float));
  s->updates = (uint64_t*)malloc(s->cap * sizeof(uint64_t));
  return s;
}

void eps_or_destroy(eps_or_store* s) {
  if (!s) return;
  omap_free(&s->index);
  free(s->keys); free(s->values); free(s->updates); free(s);
}

static float* row_ptr(const eps_or_store* s, uint64_t slot) {
  return s->values + slot * (uint64_t)s->def.dim * 3;
}

/* ShardStore::Ensure: shard_store.cpp:76-115 (home check, first-touch slot,
 * deterministic initializer, zero moments and counter). */
int64_t eps_or_ensure(eps_or_store* s, uint64_t key) {
  if (key % s->def.shard_count != s->def.shard)
    return fail(EPS_OR_INVALID_ARGUMENT, "key belongs to another shard"), -1;
  const int64_t found = omap_find(&s->index, key);
  if (found >= 0) return found;
  if (s->rows == s->cap) {
    s->cap *= 2;
    s->keys = (uint64_t*)realloc(s->keys, s->cap * sizeof(uint64_t));
    s->values = (float*)realloc(s->values, s->cap * (uint64_t)s->def.dim * 3 * sizeof(float));
    s->updates = (uint64_t*)realloc(s->updates, s->cap * sizeof(uint64_t));
  }
  const uint64_t slot = s->rows++;
  s->keys[slot] = key;
  omap_try_emplace(&s->index, key, slot);
  const uint32_t dim = s->def.dim;
  float* row = row_ptr(s, slot);
  for (uint32_t i = 0; i < dim; ++i) {
    row[i] = eps_or_init_weight(&s->def, key, i);
    row[dim + i] = row[2 * dim + i] = 0;
  }
  s->updates[slot] = 0;
  return (int64_t)slot;
}

int64_t eps_or_find(const eps_or_store* s, uint64_t key) { return omap_find(&s->index, key); }
uint64_t eps_or_row_count(const eps_or_store* s) { return s->rows; }
uint64_t eps_or_key_at(const eps_or_store* s, uint64_t slot) { return s->keys[slot]; }

/* ShardStore::Read: shard_store.cpp:117-125. */
int eps_or_read(const eps_or_store* s, uint64_t key, float* w, float* m, float* v,
                uint64_t* updates) {
  const int64_t slot = omap_find(&s->index, key);
  if (slot < 0) return fail(EPS_OR_INVALID_ARGUMENT, "unknown parameter row");
  const uint32_t dim = s->def.dim;
  const float* row = row_ptr(s, (uint64_t)slot);
  if (w) memcpy(w, row, dim * sizeof(float));
  if (m) memcpy(m, row + dim, dim * sizeof(float));
  if (v) memcpy(v, row + 2 * dim, dim * sizeof(float));
  if (updates) *updates = s->updates[slot];
  return EPS_OR_OK;
}

static void write_row(eps_or_store* s, uint64_t slot, const float* w, const float* m,
                      const float* v, uint64_t updates) {
  const uint32_t dim = s->def.dim;
  float* row = row_ptr(s, slot);
  memcpy(row, w, dim * sizeof(float));
  memcpy(row + dim, m, dim * sizeof(float));
  memcpy(row + 2 * dim, v, dim * sizeof(float));
  s->updates[slot] = updates;
}

/* ShardStore::Import: shard_store.cpp:127-138 (new row only). */
int eps_or_import(eps_or_store* s, uint64_t key, const float* w, const float* m,
                  const float* v, uint64_t updates) {
  if (omap_find(&s->index, key) >= 0) return fail(EPS_OR_INVALID_ARGUMENT, "duplicate imported row");
  const int64_t slot = eps_or_ensure(s, key);
  if (slot < 0) return EPS_OR_INVALID_ARGUMENT;
  write_row(s, (uint64_t)slot, w, m, v, updates);
  return EPS_OR_OK;
}

/* ShardStore::Overwrite: shard_store.cpp:140-149 (existing row only). */
int eps_or_overwrite(eps_or_store* s, uint64_t key, const float* w, const float* m,
                     const float* v, uint64_t updates) {
  const int64_t slot = omap_find(&s->index, key);
  if (slot < 0) return fail(EPS_OR_INVALID_ARGUMENT, "invalid returned row state");
  write_row(s, (uint64_t)slot, w, m, v, updates);
  return EPS_OR_OK;
}

/* Bulk form of Read for many keys: packed [w|m|v] rows; keys in slot order
 * when keys == NULL (first-touch order, ShardStore::keys). */
int eps_or_read_many(const eps_or_store* s, const uint64_t* keys, uint64_t count,
                     float* packed, uint64_t* updates, uint64_t* keys_out) {
  const uint32_t dim = s->def.dim;
  for (uint64_t i = 0; i < count; ++i) {
    const int64_t slot = keys ? omap_find(&s->index, keys[i]) : (int64_t)i;
    if (slot < 0 || (uint64_t)slot >= s->rows) return fail(EPS_OR_INVALID_ARGUMENT, "unknown parameter row");
    if (packed)
      memcpy(packed + i * 3 * (uint64_t)dim, row_ptr(s, (uint64_t)slot), 3 * (uint64_t)dim * sizeof(float));
    if (updates) updates[i] = s->updates[slot];
    if (keys_out) keys_out[i] = s->keys[slot];
  }
  return EPS_OR_OK;
}

void eps_or_powers(const eps_or_store* s, float* b1p, float* b2p, uint64_t* seq) {
  if (b1p) *b1p = s->beta1_power;
  if (b2p) *b2p = s->beta2_power;
  if (seq) *seq = s->optimizer_sequence;
}

/* ------------------------------------------------------------------------ */
/* ValidateFeature: src/access/batch_access.cpp:10-23. */
static int validate_feature(const eps_or_store* s, const eps_or_feature* f) {
  if (f->pooling > EPS_OR_WEIGHTED_SUM) return fail(EPS_OR_INVALID_ARGUMENT, "unsupported pooling mode");
  if (f->offsets[0] != 0 || f->offsets[f->bag_count] != f->key_count)
    return fail(EPS_OR_INVALID_ARGUMENT, "invalid bag offsets");
  for (uint64_t b = 0; b < f->bag_count; ++b) {
    if (f->offsets[b + 1] < f->offsets[b]) return fail(EPS_OR_INVALID_ARGUMENT, "invalid bag offsets");
    if (f->valid_lengths[b] < f->offsets[b + 1] - f->offsets[b])
      return fail(EPS_OR_INVALID_ARGUMENT, "original bag length is smaller than shard contribution");
  }
  if (s)
    for (uint64_t i = 0; i < f->key_count; ++i)
      if (f->keys[i] % s->def.shard_count != s->def.shard)
        return fail(EPS_OR_INVALID_ARGUMENT, "key routed to wrong shard");
  return EPS_OR_OK;
}

/* PrepareFeature: src/access/batch_access.cpp:25-52.  Dedup in first-occurrence
 * order (Ensure per new key), then per bag, per position in order,
 * dest[d] += w[d] from a zeroed output; no mean divide here.
 * Weighted-sum extension: dest[d] += w[d] * weight[i] (multiply, then add). */
int eps_or_prepare_feature(eps_or_store* s, const eps_or_feature* f,
                           uint64_t* unique_slots, uint64_t* unique_count,
                           uint64_t* occurrence_to_unique, float* contribution) {
  int rc = validate_feature(s, f);
  if (rc) return rc;
  omap unique; omap_init(&unique, f->key_count);
  uint64_t count = 0;
  for (uint64_t i = 0; i < f->key_count; ++i) {
    const int64_t prior = omap_try_emplace(&unique, f->keys[i], count);
    if (prior < 0) {
      const int64_t slot = eps_or_ensure(s, f->keys[i]);
      if (slot < 0) { omap_free(&unique); return EPS_OR_INVALID_ARGUMENT; }
      unique_slots[count] = (uint64_t)slot;
      occurrence_to_unique[i] = count++;
    } else {
      occurrence_to_unique[i] = (uint64_t)prior;
    }
  }
  omap_free(&unique);
  *unique_count = count;
  const uint32_t dim = s->def.dim;
  const uint64_t rows = f->pooling == EPS_OR_SEQUENCE ? f->key_count : f->bag_count;
  memset(contribution, 0, rows * dim * sizeof(float));
  for (uint64_t b = 0; b < f->bag_count; ++b) {
    for (uint64_t i = f->offsets[b]; i < f->offsets[b + 1]; ++i) {
      const float* w = row_ptr(s, unique_slots[occurrence_to_unique[i]]);
      float* dest = contribution + (f->pooling == EPS_OR_SEQUENCE ? i : b) * dim;
      if (f->pooling == EPS_OR_WEIGHTED_SUM) {
        const float a = f->weights[i];
        for (uint32_t d = 0; d < dim; ++d) dest[d] += w[d] * a;
      } else {
        for (uint32_t d = 0; d < dim; ++d) dest[d] += w[d];
      }
    }
  }
  return EPS_OR_OK;
}

/* Client mean: zeroed output + partial (distributed_client.cpp:113,185), then
 * values /= float(valid_length) when non-zero (distributed_client.cpp:227-232). */
void eps_or_mean_divide(float* values, const uint64_t* valid_lengths, uint64_t bags,
                        uint32_t dim) {
  for (uint64_t b = 0; b < bags; ++b) {
    for (uint32_t d = 0; d < dim; ++d) values[b * dim + d] = 0.0f + values[b * dim + d];
    if (valid_lengths[b])
      for (uint32_t d = 0; d < dim; ++d) values[b * dim + d] /= (float)valid_lengths[b];
  }
}

/* Backward scale of one occurrence: batch_access.cpp:79-80 (mean: 1.0f/len,
 * reciprocal first; else 1.0f).  Weighted-sum extension: the per-id weight. */
static float occurrence_scale(const eps_or_feature* f, uint64_t b, uint64_t i) {
  if (f->pooling == EPS_OR_WEIGHTED_SUM) return f->weights[i];
  if (f->pooling == EPS_OR_MEAN && f->valid_lengths[b]) return 1.0f / (float)f->valid_lengths[b];
  return 1.0f;
}

/* ReduceGradients for one table: src/access/batch_access.cpp:54-97.  Validate
 * every gradient value finite first; unique rows in first-occurrence order across
 * features (feature, bag, position); dest[d] += src[d] * scale (separate multiply
 * and add) from a zeroed row; then every reduced value must be finite. */
int eps_or_reduce_gradients(const eps_or_store* s, const eps_or_feature* features,
                            const float* const* gradients, uint32_t feature_count,
                            uint64_t* row_keys, float* row_values, uint64_t* row_count) {
  const uint32_t dim = s->def.dim;
  uint64_t total = 0;
  for (uint32_t fi = 0; fi < feature_count; ++fi) {
    const eps_or_feature* f = &features[fi];
    int rc = validate_feature(NULL, f);
    if (rc) return rc;
    const uint64_t rows = f->pooling == EPS_OR_SEQUENCE ? f->key_count : f->bag_count;
    for (uint64_t j = 0; j < rows * dim; ++j)
      if (!isfinite(gradients[fi][j])) return fail(EPS_OR_INVALID_ARGUMENT, "non-finite gradient");
    total += f->key_count;
  }
  omap index; omap_init(&index, total);
  uint64_t count = 0;
  for (uint32_t fi = 0; fi < feature_count; ++fi) {
    const eps_or_feature* f = &features[fi];
    for (uint64_t b = 0; b < f->bag_count; ++b) {
      for (uint64_t i = f->offsets[b]; i < f->offsets[b + 1]; ++i) {
        const float scale = occurrence_scale(f, b, i);
        int64_t u = omap_try_emplace(&index, f->keys[i], count);
        if (u < 0) {
          u = (int64_t)count++;
          row_keys[u] = f->keys[i];
          memset(row_values + (uint64_t)u * dim, 0, dim * sizeof(float));
        }
        const float* src = gradients[fi] + (f->pooling == EPS_OR_SEQUENCE ? i : b) * dim;
        float* dest = row_values + (uint64_t)u * dim;
        for (uint32_t d = 0; d < dim; ++d) dest[d] += src[d] * scale;
      }
    }
  }
  omap_free(&index);
  *row_count = count;
  for (uint64_t j = 0; j < count * dim; ++j)
    if (!isfinite(row_values[j])) return fail(EPS_OR_INVALID_ARGUMENT, "gradient reduction overflow");
  return EPS_OR_OK;
}

/* Bias-corrected step size: src/update/lazy_adam.cpp:10,27 -- float arithmetic,
 * (lr * sqrt(1 - b2p)) / (1 - b1p). */
float eps_or_lr_t(float learning_rate, float beta1_power, float beta2_power) {
  return learning_rate * sqrtf(1 - beta2_power) / (1 - beta1_power);
}

/* ValidateLazyAdam: src/update/lazy_adam.cpp:7-23. */
int eps_or_validate_lazy_adam(const eps_or_store* s, const uint64_t* keys,
                              const float* gradients, uint64_t rows) {
  const uint32_t dim = s->def.dim;
  const eps_or_table_def* o = &s->def;
  const float lr = eps_or_lr_t(o->learning_rate, s->beta1_power, s->beta2_power);
  if (!isfinite(lr)) return fail(EPS_OR_INVALID_ARGUMENT, "optimizer learning-rate overflow");
  for (uint64_t i = 0; i < rows; ++i) {
    const int64_t slot = omap_find(&s->index, keys[i]);
    if (slot < 0) return fail(EPS_OR_INVALID_ARGUMENT, "unknown parameter row");
    const float* row = row_ptr(s, (uint64_t)slot);
    for (uint32_t d = 0; d < dim; ++d) {
      const float grad = gradients[i * dim + d];
      const float m = o->beta1 * row[dim + d] + (1 - o->beta1) * grad;
      const float v = o->beta2 * row[2 * dim + d] + (1 - o->beta2) * grad * grad;
      const float w = row[d] - lr * m / (sqrtf(v) + o->epsilon);
      if (!(isfinite(m) && isfinite(v) && isfinite(w)))
        return fail(EPS_OR_INVALID_ARGUMENT, "optimizer state would overflow");
    }
  }
  return EPS_OR_OK;
}

/* ApplyLazyAdam: src/update/lazy_adam.cpp:24-42.  Per element m, v, w in that
 * order, then the clamp; ++updates per row; the table's sequence and beta powers
 * advance once per call. */
void eps_or_apply_lazy_adam(eps_or_store* s, const uint64_t* keys,
                            const float* gradients, uint64_t rows) {
  const uint32_t dim = s->def.dim;
  const eps_or_table_def* o = &s->def;
  const float lr = eps_or_lr_t(o->learning_rate, s->beta1_power, s->beta2_power);
  for (uint64_t i = 0; i < rows; ++i) {
    const int64_t slot = omap_find(&s->index, keys[i]);
    float* row = row_ptr(s, (uint64_t)slot);
    for (uint32_t d = 0; d < dim; ++d) {
      const float grad = gradients[i * dim + d];
      row[dim + d] = o->beta1 * row[dim + d] + (1 - o->beta1) * grad;
      row[2 * dim + d] = o->beta2 * row[2 * dim + d] + (1 - o->beta2) * grad * grad;
      row[d] -= lr * row[dim + d] / (sqrtf(row[2 * dim + d]) + o->epsilon);
      row[d] = bound_weight(row[d], o->bounded, o->weight_min, o->weight_max);
    }
    ++s->updates[slot];
  }
  ++s->optimizer_sequence;
  s->beta1_power *= o->beta1;
  s->beta2_power *= o->beta2;
}

/* One whole Push on CPU-owned rows: src/server/service.cpp:256-267,324-325.
 * ReduceGradients per table (every table named by a feature gets an entry),
 * ValidateLazyAdam for every table before any ApplyLazyAdam. */
int eps_or_push(eps_or_store* const* stores, uint32_t store_count,
                const eps_or_feature* features, const uint32_t* feature_store,
                const float* const* gradients, uint32_t feature_count) {
  uint64_t** keys = (uint64_t**)calloc(store_count, sizeof(uint64_t*));
  float** values = (float**)calloc(store_count, sizeof(float*));
  uint64_t* counts = (uint64_t*)calloc(store_count, sizeof(uint64_t));
  uint8_t* named = (uint8_t*)calloc(store_count, 1);
  eps_or_feature* subset = (eps_or_feature*)malloc((feature_count + 1) * sizeof(eps_or_feature));
  const float** grads = (const float**)malloc((feature_count + 1) * sizeof(float*));
  int rc = EPS_OR_OK;
  for (uint32_t t = 0; t < store_count && rc == EPS_OR_OK; ++t) {
    uint32_t n = 0;
    uint64_t total = 0;
    for (uint32_t fi = 0; fi < feature_count; ++fi)
      if (feature_store[fi] == t) {
        subset[n] = features[fi]; grads[n++] = gradients[fi]; total += features[fi].key_count;
      }
    if (!n) continue;
    named[t] = 1;
    keys[t] = (uint64_t*)malloc((total + 1) * sizeof(uint64_t));
    values[t] = (float*)malloc((total + 1) * (uint64_t)stores[t]->def.dim * sizeof(float));
    rc = eps_or_reduce_gradients(stores[t], subset, grads, n, keys[t], values[t], &counts[t]);
  }
  for (uint32_t t = 0; t < store_count && rc == EPS_OR_OK; ++t)
    if (named[t]) rc = eps_or_validate_lazy_adam(stores[t], keys[t], values[t], counts[t]);
  if (rc == EPS_OR_OK)
    for (uint32_t t = 0; t < store_count; ++t)
      if (named[t]) eps_or_apply_lazy_adam(stores[t], keys[t], values[t], counts[t]);
  for (uint32_t t = 0; t < store_count; ++t) { free(keys[t]); free(values[t]); }
  free(keys); free(values); free(counts); free(named); free(subset); free(grads);
  return rc;
}

/* ------------------------------------------------------------------------ */
/* HostCacheBackend::ApplyHost arithmetic with the caller's context powers:
 * src/cache/host_backend.cpp:119-146 (m, v, w, then the finiteness check of
 * g, w, m, v, then the clamp; all rows staged and committed only if every
 * element passes).  Arrays are row-major [rows x dim]; updated in place on
 * success only. */
int eps_or_adam_rows_ctx(float* weights, float* first, float* second,
                         const float* gradients, uint64_t rows, uint32_t dim,
                         float beta1, float beta2, float epsilon, float learning_rate,
                         float beta1_power, float beta2_power, int32_t bounded,
                         float weight_min, float weight_max) {
  if (!(beta1_power >= 0 && beta1_power < 1 && beta2_power >= 0 && beta2_power < 1 &&
        isfinite(learning_rate) && learning_rate > 0))
    return fail(EPS_OR_INVALID_ARGUMENT, "invalid cache optimizer context");
  const float lr = eps_or_lr_t(learning_rate, beta1_power, beta2_power);
  const uint64_t n = rows * dim;
  float* staged = (float*)malloc((3 * n + 1) * sizeof(float));
  float* w = staged; float* m = staged + n; float* v = staged + 2 * n;
  memcpy(w, weights, n * sizeof(float));
  memcpy(m, first, n * sizeof(float));
  memcpy(v, second, n * sizeof(float));
  for (uint64_t j = 0; j < n; ++j) {
    const float g = gradients[j];
    m[j] = beta1 * m[j] + (1 - beta1) * g;
    v[j] = beta2 * v[j] + (1 - beta2) * g * g;
    w[j] -= lr * m[j] / (sqrtf(v[j]) + epsilon);
    if (!(isfinite(g) && isfinite(w[j]) && isfinite(m[j]) && isfinite(v[j]))) {
      free(staged);
      return fail(EPS_OR_INVALID_ARGUMENT, "cached optimizer overflow");
    }
    w[j] = bound_weight(w[j], bounded, weight_min, weight_max);
  }
  memcpy(weights, w, n * sizeof(float));
  memcpy(first, m, n * sizeof(float));
  memcpy(second, v, n * sizeof(float));
  free(staged);
  return EPS_OR_OK;
}

/* HostCacheBackend::GatherHost: src/cache/host_backend.cpp:86-118.  Output
 * zeroed; UINT64_MAX occurrences skipped; per bag (or per position for
 * sequence) the unique row's weights added in occurrence order.  Weighted-sum
 * extension multiplies by the per-id weight before the add. */
int eps_or_gather_host(const eps_or_feature* f, uint32_t dim,
                       const uint64_t* occurrence_to_unique, uint64_t unique_count,
                       const float* const* unique_weights, float* out) {
  const uint64_t rows = f->pooling == EPS_OR_SEQUENCE ? f->key_count : f->bag_count;
  memset(out, 0, rows * dim * sizeof(float));
  for (uint64_t b = 0; b < f->bag_count; ++b)
    for (uint64_t i = f->offsets[b]; i < f->offsets[b + 1]; ++i) {
      const uint64_t index = occurrence_to_unique[i];
      if (index == UINT64_MAX) continue;
      if (index >= unique_count) return fail(EPS_OR_INVALID_ARGUMENT, "invalid cached occurrence map");
      const float* w = unique_weights[index];
      float* dest = out + (f->pooling == EPS_OR_SEQUENCE ? i : b) * dim;
      if (f->pooling == EPS_OR_WEIGHTED_SUM) {
        const float a = f->weights[i];
        for (uint32_t d = 0; d < dim; ++d) dest[d] += w[d] * a;
      } else {
        for (uint32_t d = 0; d < dim; ++d) dest[d] += w[d];
      }
    }
  return EPS_OR_OK;
}

/* CompactGradientBytes: src/access/compact_gradients.cpp:23-26 (RowKey is
 * 16 bytes: u32 table + padding + u64 key). */
uint64_t eps_or_compact_bytes(uint64_t rows, uint64_t source_values, uint64_t references) {
  return rows * 16 + (source_values + references) * sizeof(float) +
         ((rows + 1) + references) * sizeof(uint64_t);
}

/* ValidateCompactGradients: src/access/compact_gradients.cpp:10-22. */
int eps_or_validate_compact(uint64_t rows, const uint64_t* row_keys, uint32_t dim,
                            const float* source_values, uint64_t source_value_count,
                            const uint64_t* row_offsets, const uint64_t* source_rows,
                            const float* scales, uint64_t references) {
  if (!(dim > 0 && dim <= 4096 && rows <= (1ULL << 20)))
    return fail(EPS_OR_INVALID_ARGUMENT, "invalid compact gradient dimensions");
  if (source_value_count % dim != 0 || row_offsets[0] != 0 || row_offsets[rows] != references)
    return fail(EPS_OR_INVALID_ARGUMENT, "invalid compact gradient offsets");
  for (uint64_t r = 0; r < rows; ++r)
    if (row_offsets[r + 1] < row_offsets[r])
      return fail(EPS_OR_INVALID_ARGUMENT, "invalid compact gradient offsets");
  if (eps_or_compact_bytes(rows, source_value_count, references) > (16ULL << 20))
    return fail(EPS_OR_CAPACITY_EXCEEDED, "compact gradient exceeds byte limit");
  omap unique; omap_init(&unique, rows);
  for (uint64_t r = 0; r < rows; ++r)
    if (omap_try_emplace(&unique, row_keys[r], r) >= 0) {
      omap_free(&unique);
      return fail(EPS_OR_INVALID_ARGUMENT, "duplicate compact parameter row");
    }
  omap_free(&unique);
  const uint64_t source_count = source_value_count / dim;
  for (uint64_t j = 0; j < references; ++j)
    if (source_rows[j] >= source_count)
      return fail(EPS_OR_INVALID_ARGUMENT, "compact gradient reference is out of bounds");
  for (uint64_t j = 0; j < source_value_count; ++j)
    if (!isfinite(source_values[j])) return fail(EPS_OR_INVALID_ARGUMENT, "non-finite compact gradient value");
  for (uint64_t j = 0; j < references; ++j)
    if (!(isfinite(scales[j]) && scales[j] >= 0))
      return fail(EPS_OR_INVALID_ARGUMENT, "invalid compact gradient scale");
  return EPS_OR_OK;
}

/* ExpandCompactGradients: src/access/compact_gradients.cpp:27-39.  Per (row, d):
 * float sum = 0; sum += src[ref*dim+d] * scale[ref] over refs in order. */
int eps_or_expand_compact(uint64_t rows, const uint64_t* row_keys, uint32_t dim,
                          const float* source_values, uint64_t source_value_count,
                          const uint64_t* row_offsets, const uint64_t* source_rows,
                          const float* scales, uint64_t references, float* out) {
  int rc = eps_or_validate_compact(rows, row_keys, dim, source_values, source_value_count,
                                   row_offsets, source_rows, scales, references);
  if (rc) return rc;
  if (rows > (16ULL << 20) / (dim * 4ULL))
    return fail(EPS_OR_CAPACITY_EXCEEDED, "expanded gradient exceeds byte limit");
  for (uint64_t r = 0; r < rows; ++r)
    for (uint32_t d = 0; d < dim; ++d) {
      float sum = 0;
      for (uint64_t ref = row_offsets[r]; ref < row_offsets[r + 1]; ++ref)
        sum += source_values[source_rows[ref] * dim + d] * scales[ref];
      if (!isfinite(sum)) return fail(EPS_OR_INVALID_ARGUMENT, "compact gradient reduction overflow");
      out[r * dim + d] = sum;
    }
  return EPS_OR_OK;
}

/* BuildCompactGradients: src/access/compact_gradients.cpp:43-72.  Sources are
 * the distinct (feature, source row) pairs in first-reference order per feature;
 * references per target row keep repeats in (feature, bag, position) order.
 * Capacities: source_values >= (sum of referenced rows) * dim, source_rows and
 * scales >= total keys, row_offsets >= rows + 1. */
int eps_or_build_compact(const eps_or_feature* features, const float* const* gradients,
                         uint32_t feature_count, uint32_t dim, const uint64_t* row_keys,
                         uint64_t rows, float* source_values, uint64_t* source_value_count,
                         uint64_t* row_offsets, uint64_t* source_rows, float* scales,
                         uint64_t* references) {
  if (rows == 0) return fail(EPS_OR_INVALID_ARGUMENT, "empty compact gradient target");
  omap target; omap_init(&target, rows);
  for (uint64_t r = 0; r < rows; ++r) omap_try_emplace(&target, row_keys[r], r);
  /* Per-target reference lists, built in (feature, bag, position) order. */
  uint64_t total = 0;
  for (uint32_t fi = 0; fi < feature_count; ++fi) total += features[fi].key_count;
  uint64_t* ref_row = (uint64_t*)malloc((total + 1) * sizeof(uint64_t));
  uint64_t* ref_source = (uint64_t*)malloc((total + 1) * sizeof(uint64_t));
  float* ref_scale = (float*)malloc((total + 1) * sizeof(float));
  uint64_t nrefs = 0, nsources = 0;
  for (uint32_t fi = 0; fi < feature_count; ++fi) {
    const eps_or_feature* f = &features[fi];
    omap source_index; omap_init(&source_index, f->key_count);
    for (uint64_t b = 0; b < f->bag_count; ++b) {
      for (uint64_t i = f->offsets[b]; i < f->offsets[b + 1]; ++i) {
        const int64_t selected = omap_find(&target, f->keys[i]);
        if (selected < 0) continue;
        const uint64_t source = f->pooling == EPS_OR_SEQUENCE ? i : b;
        int64_t index = omap_try_emplace(&source_index, source, nsources);
        if (index < 0) {
          index = (int64_t)nsources++;
          memcpy(source_values + (uint64_t)index * dim, gradients[fi] + source * dim,
                 dim * sizeof(float));
        }
        ref_row[nrefs] = (uint64_t)selected;
        ref_source[nrefs] = (uint64_t)index;
        ref_scale[nrefs++] = occurrence_scale(f, b, i);
      }
    }
    omap_free(&source_index);
  }
  /* Stable grouping by target row (counting sort keeps reference order). */
  memset(row_offsets, 0, (rows + 1) * sizeof(uint64_t));
  for (uint64_t j = 0; j < nrefs; ++j) ++row_offsets[ref_row[j] + 1];
  for (uint64_t r = 0; r < rows; ++r) row_offsets[r + 1] += row_offsets[r];
  uint64_t* cursor = (uint64_t*)malloc((rows + 1) * sizeof(uint64_t));
  memcpy(cursor, row_offsets, (rows + 1) * sizeof(uint64_t));
  for (uint64_t j = 0; j < nrefs; ++j) {
    const uint64_t at = cursor[ref_row[j]]++;
    source_rows[at] = ref_source[j];
    scales[at] = ref_scale[j];
  }
  free(cursor); free(ref_row); free(ref_source); free(ref_scale); omap_free(&target);
  *source_value_count = nsources * dim;
  *references = nrefs;
  return eps_or_validate_compact(rows, row_keys, dim, source_values, nsources * dim,
                                 row_offsets, source_rows, scales, nrefs);
}

/* ------------------------------------------------------------------------ */
/* Snapshot format: src/store/snapshot.cpp.  Little-endian u64 and float
 * fields, strings as a u64 length plus bytes, FNV-1a over every byte before
 * the trailing checksum (Binary::Bytes/U64/Float/String, :29-76). */
#define FNV_PRIME 1099511628211ULL
#define SNAPSHOT_MAGIC_V1 0x3153504541524853ULL
#define SNAPSHOT_MAGIC_V2 0x3253504541524853ULL

uint64_t eps_or_fnv1a(uint64_t hash, const void* data, uint64_t size) {
  const unsigned char* p = (const unsigned char*)data;
  for (uint64_t i = 0; i < size; ++i) hash = (hash ^ p[i]) * FNV_PRIME;
  return hash;
}

typedef struct snap_io {
  FILE* f;
  uint64_t hash;
  int failed;
} snap_io;

static void snap_put(snap_io* io, const void* data, uint64_t size, int hashed) {
  if (fwrite(data, 1, size, io->f) != size) io->failed = 1;
  if (hashed) io->hash = eps_or_fnv1a(io->hash, data, size);
}
static void snap_u64(snap_io* io, uint64_t v, int hashed) {
  unsigned char b[8];
  for (int i = 0; i < 8; ++i) b[i] = (unsigned char)(v >> (8 * i));
  snap_put(io, b, 8, hashed);
}
static void snap_f32(snap_io* io, float x) {
  uint32_t u;
  memcpy(&u, &x, 4);
  unsigned char b[4];
  for (int i = 0; i < 4; ++i) b[i] = (unsigned char)(u >> (8 * i));
  snap_put(io, b, 4, 1);
}
static int snap_get(snap_io* io, void* data, uint64_t size, int hashed) {
  if (fread(data, 1, size, io->f) != size) return io->failed = 1, 0;
  if (hashed) io->hash = eps_or_fnv1a(io->hash, data, size);
  return 1;
}
static uint64_t snap_get_u64(snap_io* io, int hashed) {
  unsigned char b[8] = {0};
  snap_get(io, b, 8, hashed);
  uint64_t v = 0;
  for (int i = 0; i < 8; ++i) v |= (uint64_t)b[i] << (8 * i);
  return v;
}
static float snap_get_f32(snap_io* io) {
  unsigned char b[4] = {0};
  snap_get(io, b, 4, 1);
  uint32_t u = 0;
  for (int i = 0; i < 4; ++i) u |= (uint32_t)b[i] << (8 * i);
  float x;
  memcpy(&x, &u, 4);
  return x;
}

/* Binary::Definition (:77-98): id, dimension, shard count, partition epoch,
 * the six optimizer floats, [bounds flag (+ min, max) in format 2], the
 * initializer bounds and seed. */
static void snap_put_definition(snap_io* io, const eps_or_table_def* d, uint64_t epoch) {
  snap_u64(io, d->id, 1);
  snap_u64(io, d->dim, 1);
  snap_u64(io, d->shard_count, 1);
  snap_u64(io, epoch, 1);
  snap_f32(io, d->learning_rate); snap_f32(io, d->beta1); snap_f32(io, d->beta2);
  snap_f32(io, d->epsilon); snap_f32(io, d->initial_beta1_power); snap_f32(io, d->initial_beta2_power);
  snap_u64(io, d->bounded ? 1 : 0, 1);
  if (d->bounded) { snap_f32(io, d->weight_min); snap_f32(io, d->weight_max); }
  snap_f32(io, d->init_min); snap_f32(io, d->init_max);
  snap_u64(io, d->init_seed, 1);
}

int eps_or_snapshot_write(const char* path, const char* run, uint64_t shard,
                          uint64_t shard_count, uint64_t epoch, eps_or_store* const* stores,
                          uint32_t table_count) {
  snap_io io = {fopen(path, "wb"), EPS_OR_FNV_OFFSET, 0};
  if (!io.f) return fail(EPS_OR_UNAVAILABLE, "cannot create snapshot");
  snap_u64(&io, SNAPSHOT_MAGIC_V2, 1);
  const uint64_t run_bytes = strlen(run);
  snap_u64(&io, run_bytes, 1);
  snap_put(&io, run, run_bytes, 1);
  snap_u64(&io, shard, 1); snap_u64(&io, shard_count, 1); snap_u64(&io, epoch, 1);
  snap_u64(&io, table_count, 1);
  for (uint32_t t = 0; t < table_count; ++t) {
    const eps_or_store* s = stores[t];
    snap_put_definition(&io, &s->def, epoch);
    snap_u64(&io, s->optimizer_sequence, 1);
    snap_f32(&io, s->beta1_power);
    snap_f32(&io, s->beta2_power);
    snap_u64(&io, s->rows, 1);
    const uint64_t n = (uint64_t)s->def.dim * 3;
    for (uint64_t r = 0; r < s->rows; ++r) {
      snap_u64(&io, s->keys[r], 1);
      snap_u64(&io, s->updates[r], 1);
      const float* row = row_ptr(s, r);
      for (uint64_t i = 0; i < n; ++i) snap_f32(&io, row[i]);
    }
  }
  snap_u64(&io, io.hash, 0);
  if (fclose(io.f) != 0) io.failed = 1;
  return io.failed ? fail(EPS_OR_UNAVAILABLE, "snapshot write failed") : EPS_OR_OK;
}

int eps_or_snapshot_read(const char* path, char* run, uint64_t run_capacity, uint64_t* shard,
                         uint64_t* shard_count, uint64_t* epoch, uint32_t* version,
                         eps_or_store** stores, uint32_t capacity, uint32_t* table_count,
                         uint64_t* checksum) {
  snap_io io = {fopen(path, "rb"), EPS_OR_FNV_OFFSET, 0};
  if (!io.f) return fail(EPS_OR_UNAVAILABLE, "cannot open snapshot");
  uint32_t made = 0;
  int rc = EPS_OR_OK;
  const uint64_t magic = snap_get_u64(&io, 1);
  if (magic != SNAPSHOT_MAGIC_V1 && magic != SNAPSHOT_MAGIC_V2) {
    rc = fail(EPS_OR_INVALID_ARGUMENT, "unsupported snapshot format");
    goto done;
  }
  *version = magic == SNAPSHOT_MAGIC_V2 ? 2 : 1;
  const uint64_t run_bytes = snap_get_u64(&io, 1);
  if (run_bytes > 1024 || run_bytes + 1 > run_capacity) {
    rc = fail(EPS_OR_INVALID_ARGUMENT, "snapshot string too long");
    goto done;
  }
  snap_get(&io, run, run_bytes, 1);
  run[run_bytes] = 0;
  *shard = snap_get_u64(&io, 1); *shard_count = snap_get_u64(&io, 1); *epoch = snap_get_u64(&io, 1);
  const uint64_t tables = snap_get_u64(&io, 1);
  if (tables > capacity || tables > 1024) {
    rc = fail(EPS_OR_INVALID_ARGUMENT, "snapshot table count exceeds limit");
    goto done;
  }
  for (uint64_t t = 0; t < tables && !io.failed; ++t) {
    eps_or_table_def d;
    memset(&d, 0, sizeof d);
    d.id = (uint32_t)snap_get_u64(&io, 1);
    d.dim = (uint32_t)snap_get_u64(&io, 1);
    d.shard_count = (uint32_t)snap_get_u64(&io, 1);
    d.shard = (uint32_t)*shard;
    const uint64_t table_epoch = snap_get_u64(&io, 1);
    d.learning_rate = snap_get_f32(&io); d.beta1 = snap_get_f32(&io); d.beta2 = snap_get_f32(&io);
    d.epsilon = snap_get_f32(&io); d.initial_beta1_power = snap_get_f32(&io);
    d.initial_beta2_power = snap_get_f32(&io);
    if (*version == 2) {
      const uint64_t enabled = snap_get_u64(&io, 1);
      if (enabled > 1) { rc = fail(EPS_OR_INVALID_ARGUMENT, "invalid snapshot weight-bounds flag"); goto done; }
      d.bounded = (int32_t)enabled;
      if (enabled) { d.weight_min = snap_get_f32(&io); d.weight_max = snap_get_f32(&io); }
    }
    d.init_min = snap_get_f32(&io); d.init_max = snap_get_f32(&io);
    d.init_seed = snap_get_u64(&io, 1);
    if (d.dim == 0 || d.dim > 65536 || d.shard_count != *shard_count || table_epoch != *epoch) {
      rc = fail(EPS_OR_INVALID_ARGUMENT, "table partition does not match snapshot");
      goto done;
    }
    eps_or_store* s = eps_or_create(&d);
    if (!s) { rc = EPS_OR_INVALID_ARGUMENT; goto done; }
    stores[made++] = s;
    s->optimizer_sequence = snap_get_u64(&io, 1);
    s->beta1_power = snap_get_f32(&io);
    s->beta2_power = snap_get_f32(&io);
    const uint64_t rows = snap_get_u64(&io, 1);
    const uint32_t dim = d.dim;
    float* buf = (float*)malloc((uint64_t)dim * 3 * sizeof(float));
    for (uint64_t r = 0; r < rows && !io.failed; ++r) {
      const uint64_t key = snap_get_u64(&io, 1), updates = snap_get_u64(&io, 1);
      for (uint64_t i = 0; i < (uint64_t)dim * 3; ++i) buf[i] = snap_get_f32(&io);
      if (!io.failed && eps_or_import(s, key, buf, buf + dim, buf + 2 * dim, updates)) {
        rc = EPS_OR_INVALID_ARGUMENT;
        free(buf);
        goto done;
      }
    }
    free(buf);
  }
  {
    const uint64_t actual = io.hash;
    const uint64_t expected = snap_get_u64(&io, 0);
    unsigned char extra;
    if (io.failed) rc = fail(EPS_OR_UNAVAILABLE, "snapshot truncated");
    else if (actual != expected) rc = fail(EPS_OR_INVALID_ARGUMENT, "snapshot checksum mismatch");
    else if (fread(&extra, 1, 1, io.f) == 1) rc = fail(EPS_OR_INVALID_ARGUMENT, "snapshot contains trailing data");
    *checksum = expected;
  }
done:
  fclose(io.f);
  *table_count = made;
  if (rc != EPS_OR_OK) {
    for (uint32_t i = 0; i < made; ++i) eps_or_destroy(stores[i]);
    *table_count = 0;
  }
  return rc;
}
