/*
 * mdl_oracle.c -- CPU restatement of the reference sparse path (TEST
 * INFRASTRUCTURE ONLY: used by tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py as the checker, never by the product).
 *
 * Every function restates the reference semantics in plain C with fp64
 * accumulation, rounding only where the reference stores a value:
 *
 *   oracle_bucketize_pre_hashed  src/features.py:360-376, src/dataloader.py:8463-8493
 *   oracle_bucketize_mod         src/benchmark.py:1246-1250 (Python floor-mod)
 *   oracle_pool                  src/model.py:509-570 (mean; sum = the same
 *                                without the division, F.embedding_bag(sum))
 *   oracle_coalesce              torch sparse coalesce used at src/optim.py:323-324
 *   oracle_rowwise_adagrad       src/optim.py:31-62 (Triton kernel) + :345-357
 *   oracle_sparse_step           the whole fwd + bwd + update step of one
 *                                grouped batch (timed as the CPU baseline)
 *
 * Pinning of each function is listed in the header of oracle/oracle.py.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------- bucketing */

int64_t oracle_bucketize_pre_hashed(const int64_t* raw, const uint8_t* valid, int64_t n,
                                    int64_t num_buckets, int64_t* out) {
  int64_t zeros = 0;
  for (int64_t i = 0; i < n; ++i) {
    if (valid && !valid[i]) {
      out[i] = 0;
      continue;
    }
    uint64_t u = (uint64_t)raw[i];
    out[i] = (int64_t)((u & (uint64_t)(num_buckets - 1)) + 1);
    zeros += raw[i] == 0;
  }
  return zeros;
}

static int64_t floormod(int64_t a, int64_t m) {
  int64_t r = a % m;
  return r < 0 ? r + m : r;
}

void oracle_bucketize_mod(const int64_t* raw, const uint8_t* valid, int64_t n, int64_t num_embeddings,
                          int64_t* out) {
  const int64_t m = num_embeddings - 1;
  for (int64_t i = 0; i < n; ++i) {
    if (valid && !valid[i]) {
      out[i] = 0;
      continue;
    }
    /* (raw - 1) mod m == ((raw mod m) - 1) mod m, without int64 overflow */
    out[i] = 1 + floormod(floormod(raw[i], m) - 1, m);
  }
}

/* -------------------------------------------------------------- pooling */

/* mode 0: no pooling (out row i = W[ids[i]]), 1: sum, 2: mean.
 * W is fp32 [rows, dim]; out fp64 [nb, dim]; count fp64 [nb] = sum of w_i. */
void oracle_pool(const float* W, int64_t rows, int32_t dim, const int64_t* ids, const int64_t* offsets,
                 int64_t nb, int32_t mode, int32_t exclude, double* out, double* count) {
  for (int64_t b = 0; b < nb; ++b) {
    double* o = out + b * dim;
    for (int32_t j = 0; j < dim; ++j) o[j] = 0.0;
    double c = 0.0;
    for (int64_t i = offsets[b]; i < offsets[b + 1]; ++i) {
      const int64_t id = ids[i];
      const double w = (exclude && id == 0) ? 0.0 : 1.0;
      if (id < 0 || id >= rows) continue;
      c += w;
      if (w == 0.0) continue;
      const float* r = W + id * dim;
      for (int32_t j = 0; j < dim; ++j) o[j] += (double)r[j];
    }
    if (count) count[b] = c;
    if (mode == 2) {
      const double den = c < 1.0 ? 1.0 : c;
      for (int32_t j = 0; j < dim; ++j) o[j] /= den;
    }
  }
}

/* ------------------------------------------------------------- coalesce */

typedef struct {
  int64_t row;
  int64_t pos;
} pair_t;

static int cmp_pair(const void* a, const void* b) {
  const pair_t* x = (const pair_t*)a;
  const pair_t* y = (const pair_t*)b;
  if (x->row != y->row) return x->row < y->row ? -1 : 1;
  return x->pos < y->pos ? -1 : (x->pos > y->pos);
}

/* Rows ascending and unique; values summed in fp64 in input order. */
int64_t oracle_coalesce(const int64_t* rows, const double* vals, int64_t n, int32_t dim, int64_t* out_rows,
                        double* out_vals) {
  pair_t* p = (pair_t*)malloc(sizeof(pair_t) * (size_t)(n > 0 ? n : 1));
  for (int64_t i = 0; i < n; ++i) {
    p[i].row = rows[i];
    p[i].pos = i;
  }
  qsort(p, (size_t)n, sizeof(pair_t), cmp_pair);
  int64_t u = -1;
  for (int64_t i = 0; i < n; ++i) {
    if (i == 0 || p[i].row != p[i - 1].row) {
      ++u;
      out_rows[u] = p[i].row;
      for (int32_t j = 0; j < dim; ++j) out_vals[u * dim + j] = 0.0;
    }
    const double* v = vals + p[i].pos * dim;
    for (int32_t j = 0; j < dim; ++j) out_vals[u * dim + j] += v[j];
  }
  free(p);
  return u + 1;
}

/* -------------------------------------------------------------- adagrad */

static float bf16_round(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) {
    u |= 0x00400000u;
  } else {
    u += 0x7fffu + ((u >> 16) & 1u);
  }
  u &= 0xffff0000u;
  float r;
  memcpy(&r, &u, 4);
  return r;
}

/* W holds fp32 values (bf16 tables are passed widened; is_bf16 rounds the
 * stored result to bf16, round-to-nearest-even).  acc fp32 [num_rows].
 * Rows must be unique, as the reference kernel requires. */
void oracle_rowwise_adagrad(float* W, int32_t is_bf16, int64_t num_rows, int32_t dim, float* acc,
                            const int64_t* rows, int64_t n, const double* vals, double lr, double eps) {
  for (int64_t i = 0; i < n; ++i) {
    const int64_t r = rows[i];
    if (r < 0 || r >= num_rows) continue;
    const double* g = vals + i * dim;
    double ss = 0.0;
    for (int32_t j = 0; j < dim; ++j) ss += g[j] * g[j];
    const float a = (float)((double)acc[r] + ss / (double)dim);
    acc[r] = a;
    const double den = sqrt((double)a) + eps;
    float* w = W + r * dim;
    for (int32_t j = 0; j < dim; ++j) {
      float nw = (float)((double)w[j] - lr * (g[j] / den));
      w[j] = is_bf16 ? bf16_round(nw) : nw;
    }
  }
}

/* ---------------------------------------------------------- sparse step */

/*
 * One fwd + bwd + row-wise Adagrad step over F features reading T tables.
 *   feature f: table[f], pooling[f] (0 none, 1 sum, 2 mean), exclude[f],
 *              ids + ids_off[f] .. ids_off[f+1], bag offsets (relative to the
 *              feature's first id) at offs + bag_off[f] (num_bags[f]+1 entries;
 *              unused for pooling 0, where every id is one output row),
 *              output rows at out + out_col[f] with row stride out_stride,
 *              upstream gradient at grad + out_col[f] (same layout).
 *   table t: W[t] fp32 [rows[t], dims[t]], acc[t] fp32 [rows[t]].
 * Per-id gradient: grad[bag] / max(count, 1) (mean) or grad[bag]; padding
 * id 0 and nulls under "exclude" get none.  Duplicates summed in fp64.
 */
void oracle_sparse_step(int32_t F, const int32_t* table, const int32_t* pooling, const int32_t* exclude,
                        const int64_t* ids, const int64_t* ids_off, const int64_t* offs, const int64_t* bag_off,
                        const int64_t* num_bags, const int64_t* out_col, int64_t out_stride, double* out,
                        const double* grad, int32_t T, float** W, float** acc, const int64_t* rows,
                        const int32_t* dims, const int32_t* is_bf16, double lr, double eps) {
  for (int32_t t = 0; t < T; ++t) {
    const int32_t dim = dims[t];
    /* gather every contribution to table t */
    int64_t total = 0;
    for (int32_t f = 0; f < F; ++f)
      if (table[f] == t) total += ids_off[f + 1] - ids_off[f];
    int64_t* crow = (int64_t*)malloc(sizeof(int64_t) * (size_t)(total > 0 ? total : 1));
    double* cval = (double*)malloc(sizeof(double) * (size_t)(total > 0 ? total : 1) * dim);
    int64_t k = 0;
    for (int32_t f = 0; f < F; ++f) {
      if (table[f] != t) continue;
      const int64_t* fid = ids + ids_off[f];
      const int64_t nid = ids_off[f + 1] - ids_off[f];
      double* fo = out + out_col[f];
      const double* fg = grad + out_col[f];
      if (pooling[f] == 0) {
        for (int64_t i = 0; i < nid; ++i) {
          const int64_t id = fid[i];
          for (int32_t j = 0; j < dim; ++j)
            fo[i * out_stride + j] = (id >= 0 && id < rows[t]) ? (double)W[t][id * dim + j] : 0.0;
          if (id <= 0 || id >= rows[t]) continue; /* padding 0 gets no gradient */
          crow[k] = id;
          for (int32_t j = 0; j < dim; ++j) cval[k * dim + j] = fg[i * out_stride + j];
          ++k;
        }
      } else {
        const int64_t* bo = offs + bag_off[f];
        for (int64_t b = 0; b < num_bags[f]; ++b) {
          double c = 0.0;
          double* o = fo + b * out_stride;
          for (int32_t j = 0; j < dim; ++j) o[j] = 0.0;
          for (int64_t i = bo[b]; i < bo[b + 1]; ++i) {
            const int64_t id = fid[i];
            if (id < 0 || id >= rows[t]) continue;
            const double w = (exclude[f] && id == 0) ? 0.0 : 1.0;
            c += w;
            if (w == 0.0) continue;
            for (int32_t j = 0; j < dim; ++j) o[j] += (double)W[t][id * dim + j];
          }
          const double den = (pooling[f] == 2) ? (c < 1.0 ? 1.0 : c) : 1.0;
          if (pooling[f] == 2)
            for (int32_t j = 0; j < dim; ++j) o[j] /= den;
          const double* g = fg + b * out_stride;
          for (int64_t i = bo[b]; i < bo[b + 1]; ++i) {
            const int64_t id = fid[i];
            if (id <= 0 || id >= rows[t]) continue;
            crow[k] = id;
            for (int32_t j = 0; j < dim; ++j) cval[k * dim + j] = g[j] / den;
            ++k;
          }
        }
      }
    }
    int64_t* urow = (int64_t*)malloc(sizeof(int64_t) * (size_t)(k > 0 ? k : 1));
    double* uval = (double*)malloc(sizeof(double) * (size_t)(k > 0 ? k : 1) * dim);
    const int64_t u = oracle_coalesce(crow, cval, k, dim, urow, uval);
    oracle_rowwise_adagrad(W[t], is_bf16[t], rows[t], dim, acc[t], urow, u, uval, lr, eps);
    free(crow);
    free(cval);
    free(urow);
    free(uval);
  }
}
