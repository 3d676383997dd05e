// Backward of the grouped lookup: sort, unique and deterministic segment
// reduction of per-id gradients, fused with the row-wise Adagrad update (or
// writing a coalesced sparse gradient).
//
// After the stable radix sort every distinct (table, row) is one run of equal
// keys whose payloads (gradient rows) appear in input order.  The sorted
// array is cut into chunks of <= kChunk entries that never straddle two
// tables; one wavefront reduces one chunk with the same slot-parallel
// segmented scan as the forward pooling.  A run that ends inside the chunk it
// started in is finished there: its summed gradient goes straight into the
// Adagrad update (weights and accumulator read and written once) or into the
// coalesced gradient.  A run that crosses chunk boundaries (hot Zipf rows can
// have 10^4+ entries) leaves one fp32 partial per chunk it touches; a second
// kernel adds those partials in chunk order and finishes the run.  No
// floating-point atomics are used, so results do not depend on scheduling.
#include "common.cuh"

namespace mdl {

int sort_pairs(uint32_t* keys, uint32_t* vals, uint32_t* keys_alt, uint32_t* vals_alt, int64_t n,
               int key_bits, void* ws, size_t ws_bytes, int* in_alt, hipStream_t s);
size_t sort_ws_bytes(int64_t n);
int launch_sum_partials(const float* partial, int64_t m, const int64_t* m_dev, float* out, hipStream_t s);

constexpr int kChunkMax = 512;
constexpr int kBwdWaves = 4;
constexpr int kPlanThreads = 1024;

enum { kHeadOpen = 1, kTailOpen = 2, kSingle = 4 };
// Adagrad: update the rows; Coalesce: write the coalesced gradient; Sumsq:
// only the squared 2-norm of the coalesced gradient (for clipping).
enum { kModeAdagrad = 0, kModeCoalesce = 1, kModeSumsq = 2 };

struct BwdWs {
  uint32_t* keys_alt;
  uint32_t* vals_alt;
  void* sort_ws;
  size_t sort_bytes;
  int64_t* table_start;   // [T]
  int64_t* table_end;     // [T]
  int64_t* chunk_base;    // [T+1]
  int64_t* table_cb;      // [T] entries per chunk of table t
  int32_t* chunk_flags;   // [max_chunks]
  int64_t* head_base;     // [max_chunks+1]
  void* scan_ws;
  size_t scan_bytes;
  float* part_first;      // [max_chunks, max_dim]
  float* part_last;       // [max_chunks, max_dim]
  float* chunk_ss;        // [max_chunks] squared norms of the runs finished per chunk
};

// Chunks hold kPassesPerChunk passes of G rows; G >= 1, so a table of m
// entries has at most ceil(m / kPassesPerChunk) chunks.
static inline int64_t max_chunks_for(int64_t n, int32_t T) {
  return (n + kPassesPerChunk - 1) / kPassesPerChunk + T + 1;
}

static size_t carve(BwdWs* w, void* base, int64_t n, int32_t T, int32_t max_dim) {
  char* p = static_cast<char*>(base);
  const char* start = p;
  auto take = [&](size_t bytes) {
    char* r = p;
    p += (bytes + 255) & ~size_t(255);
    return r;
  };
  const int64_t nn = n > 0 ? n : 1;
  const int64_t mc = max_chunks_for(n, T);
  w->keys_alt = (uint32_t*)take(nn * 4);
  w->vals_alt = (uint32_t*)take(nn * 4);
  w->sort_bytes = sort_ws_bytes(nn);
  w->sort_ws = take(w->sort_bytes);
  w->table_start = (int64_t*)take((size_t)T * 8 + 8);
  w->table_end = (int64_t*)take((size_t)T * 8 + 8);
  w->chunk_base = (int64_t*)take(((size_t)T + 1) * 8);
  w->table_cb = (int64_t*)take((size_t)T * 8 + 8);
  w->chunk_flags = (int32_t*)take((size_t)mc * 4);
  w->head_base = (int64_t*)take(((size_t)mc + 1) * 8);
  w->scan_bytes = mdl_offsets_workspace_bytes(mc);
  w->scan_ws = take(w->scan_bytes);
  w->part_first = (float*)take((size_t)mc * max_dim * 4);
  w->part_last = (float*)take((size_t)mc * max_dim * 4);
  w->chunk_ss = (float*)take((size_t)mc * 4);
  return (size_t)(p - start);
}

// ------------------------------------------------------------------ plan --

__device__ __forceinline__ int64_t lower_bound_u32(const uint32_t* a, int64_t n, uint64_t x) {
  int64_t lo = 0, hi = n;
  while (lo < hi) {
    const int64_t mid = (lo + hi) >> 1;
    if ((uint64_t)a[mid] < x) lo = mid + 1;
    else hi = mid;
  }
  return lo;
}

// Whether a table's rows (and so its gradient and value rows, which the host
// lays out alike) use 16-byte vectors, and the chunk length that gives one
// wave kPassesPerChunk passes over it.
__device__ __forceinline__ bool table_vec(const mdl_table& tb) {
  return table_vec_of(tb.weight, tb.dim, tb.wdtype);
}

__device__ __forceinline__ int64_t table_chunk_len(const mdl_table& tb) {
  const int c = table_vec(tb) ? (tb.wdtype == MDL_BF16 ? 8 : 4) : 1;
  const int64_t g = kWave / lanes_for(tb.dim > 0 ? tb.dim : 1, c);
  const int64_t cb = (int64_t)kPassesPerChunk * g;
  return cb < kChunkMax ? cb : kChunkMax;
}

__global__ __launch_bounds__(kPlanThreads) void bwd_plan_kernel(const mdl_table* __restrict__ tables, int32_t T,
                                                                 const uint32_t* __restrict__ keys, int64_t n,
                                                                 int64_t* table_start, int64_t* table_end,
                                                                 int64_t* chunk_base, int64_t* table_cb) {
  __shared__ int64_t smem[kPlanThreads];
  int64_t carry = 0;
  for (int32_t base = 0; base < T; base += kPlanThreads) {
    const int32_t t = base + threadIdx.x;
    int64_t nch = 0;
    if (t < T) {
      const uint64_t lo_key = (uint64_t)tables[t].row_base;
      const uint64_t hi_key = lo_key + (uint64_t)tables[t].num_rows;
      const int64_t lo = lower_bound_u32(keys, n, lo_key);
      const int64_t hi = lower_bound_u32(keys, n, hi_key);
      table_start[t] = lo;
      table_end[t] = hi;
      const int64_t cb = table_chunk_len(tables[t]);
      table_cb[t] = cb;
      nch = (hi - lo + cb - 1) / cb;
    }
    smem[threadIdx.x] = nch;
    __syncthreads();
    for (int d = 1; d < kPlanThreads; d <<= 1) {
      int64_t o = threadIdx.x >= d ? smem[threadIdx.x - d] : 0;
      __syncthreads();
      smem[threadIdx.x] += o;
      __syncthreads();
    }
    if (t < T) chunk_base[t] = carry + smem[threadIdx.x] - nch;
    carry += smem[kPlanThreads - 1];
    __syncthreads();
  }
  if (threadIdx.x == 0) chunk_base[T] = carry;
}

// Heads (first entry of a run) per chunk, for the coalesced layout.
struct ChunkRange {
  int64_t c_begin, c_end, t_begin, t_end;
  int32_t t;
};

__device__ __forceinline__ int64_t uni64b(int64_t v) {
  int lo = __builtin_amdgcn_readfirstlane((int)(v & 0xffffffff));
  int hi = __builtin_amdgcn_readfirstlane((int)(v >> 32));
  return (int64_t)(((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo);
}

// Locate chunk c: returns false when c is past the last chunk.
__device__ __forceinline__ bool find_chunk(int64_t c, int32_t T, const int64_t* chunk_base,
                                           const int64_t* table_start, const int64_t* table_end,
                                           const int64_t* table_cb, ChunkRange* r) {
  const int64_t total = chunk_base[T];
  if (c >= total) return false;
  int32_t lo = 0, hi = T - 1;  // last t with chunk_base[t] <= c
  while (lo < hi) {
    const int32_t mid = (lo + hi + 1) >> 1;
    if (chunk_base[mid] <= c) lo = mid;
    else hi = mid - 1;
  }
  // Skip empty tables that share the same chunk_base.
  while (lo + 1 <= T - 1 && chunk_base[lo + 1] <= c) ++lo;
  r->t = __builtin_amdgcn_readfirstlane(lo);
  r->t_begin = uni64b(table_start[lo]);
  r->t_end = uni64b(table_end[lo]);
  const int64_t cb = uni64b(table_cb[lo]);
  r->c_begin = r->t_begin + (c - chunk_base[lo]) * cb;
  r->c_end = r->c_begin + cb < r->t_end ? r->c_begin + cb : r->t_end;
  r->c_begin = uni64b(r->c_begin);
  r->c_end = uni64b(r->c_end);
  return true;
}

__global__ __launch_bounds__(256) void count_heads_kernel(int32_t T, const int64_t* chunk_base,
                                                          const int64_t* table_start, const int64_t* table_end,
                                                          const int64_t* table_cb,
                                                          const uint32_t* __restrict__ keys, int64_t max_chunks,
                                                          int64_t* __restrict__ heads) {
  const int w = threadIdx.x / kWave, lane = lane_id();
  const int64_t c = uni64b((int64_t)blockIdx.x * 4 + w);
  if (c >= max_chunks) return;
  ChunkRange r;
  if (!find_chunk(c, T, chunk_base, table_start, table_end, table_cb, &r)) {
    if (lane == 0) heads[c] = 0;
    return;
  }
  int cnt = 0;
  for (int64_t e = r.c_begin + lane; e < r.c_end; e += kWave)
    cnt += (e == r.t_begin || keys[e] != keys[e - 1]) ? 1 : 0;
  for (int m = 1; m < kWave; m <<= 1) cnt += __shfl_xor(cnt, m);
  if (lane == 0) heads[c] = cnt;
}

__global__ void unique_range_kernel(int32_t T, const int64_t* chunk_base, const int64_t* head_base,
                                    int64_t* unique_range) {
  for (int32_t t = blockIdx.x * blockDim.x + threadIdx.x; t < T; t += gridDim.x * blockDim.x) {
    unique_range[2 * t] = head_base[chunk_base[t]];
    unique_range[2 * t + 1] = head_base[chunk_base[t + 1]];
  }
}

__global__ void unique_range_zero(int32_t T, int64_t* unique_range) {
  for (int32_t t = blockIdx.x * blockDim.x + threadIdx.x; t < 2 * T; t += gridDim.x * blockDim.x)
    unique_range[t] = 0;
}

// Keys of an arbitrary row-index list (an uncoalesced COO gradient).
__global__ void sparse_keys_kernel(const int64_t* __restrict__ ids, int64_t n, int64_t num_rows, int64_t row_base,
                                   int64_t payload_base, int64_t padding_idx, uint32_t* __restrict__ keys,
                                   uint32_t* __restrict__ payload, uint32_t sentinel, int32_t* error_count) {
  int bad = 0;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t id = ids[i];
    const bool in_range = (uint64_t)id < (uint64_t)num_rows;
    bad += !in_range;
    keys[i] = (in_range && id != padding_idx) ? (uint32_t)(row_base + id) : sentinel;
    payload[i] = (uint32_t)(payload_base + i);
  }
  if (bad && error_count) atomicAdd(error_count, bad);
}

// -------------------------------------------------------------- reduce --

struct BwdArgs {
  const mdl_feature* feats;
  int32_t F;
  const mdl_table* tables;
  int32_t T;
  const uint32_t* keys;
  const uint32_t* vals;
  const float* bag_count;
  const int64_t* table_start;
  const int64_t* table_end;
  const int64_t* chunk_base;
  const int64_t* table_cb;
  int32_t* chunk_flags;
  const int64_t* head_base;
  float* part_first;
  float* part_last;
  float* chunk_ss;
  const float* grad_scale;  // Adagrad: gradients are multiplied by *grad_scale (NULL: 1)
  int64_t max_chunks;
  int32_t max_dim;
  float lr, eps;
  int32_t mode;
  const uint64_t* rows_addr;
  const uint64_t* values_addr;
  const int64_t* unique_range;
};

// Feature that owns gradient payload p: the last feature whose
// payload_base <= p (descriptors are ordered by payload_base).
__device__ __forceinline__ int32_t feature_of(const BwdArgs& a, int32_t single, uint32_t p) {
  if (single >= 0) return single;
  int32_t lo = 0, hi = a.F - 1;
  while (lo < hi) {
    const int32_t mid = (lo + hi + 1) >> 1;
    if ((uint64_t)a.feats[mid].payload_base <= (uint64_t)p) lo = mid;
    else hi = mid - 1;
  }
  return lo;
}

template <int kMode, typename TW, typename TG, int C>
struct Reducer {
  const BwdArgs& a;
  int32_t t;
  int dim, L, G, slot, sub, col;
  bool col_ok;
  int32_t single;
  TW* W;
  float* state;
  int64_t row_base;
  // fields of the table's only feature (single >= 0)
  const TG* g_base;
  int64_t g_stride, pbase;
  bool g_mean;
  float scale;

  __device__ Reducer(const BwdArgs& args, int32_t table) : a(args), t(table) {
    const mdl_table& tb = a.tables[t];
    dim = __builtin_amdgcn_readfirstlane(tb.dim);
    single = __builtin_amdgcn_readfirstlane(tb.feature);
    W = (TW*)uni64b((int64_t)tb.weight);
    state = (float*)uni64b((int64_t)tb.state);
    row_base = uni64b(tb.row_base);
    L = lanes_for(dim, C);
    G = kWave / L;
    const int lane = lane_id();
    slot = lane / L;
    sub = lane % L;
    col = sub * C;
    col_ok = col < dim;
    g_base = nullptr;
    g_stride = pbase = 0;
    g_mean = false;
    scale = 1.f;
    if (kMode == kModeAdagrad && a.grad_scale != nullptr)
      scale = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, *a.grad_scale)));
    if (single >= 0) {
      const mdl_feature& f = a.feats[single];
      g_base = (const TG*)uni64b((int64_t)f.grad);
      g_stride = uni64b(f.out_stride);
      pbase = uni64b(f.payload_base);
      g_mean = __builtin_amdgcn_readfirstlane(f.pooling) == MDL_POOL_MEAN;
    }
  }

  // Gradient row of payload p and whether it is divided by its bag count.
  __device__ __forceinline__ const TG* grad_row(uint32_t p, bool& mean) const {
    if (single >= 0) {
      mean = g_mean;
      return g_base + ((int64_t)p - pbase) * g_stride;
    }
    const mdl_feature& f = a.feats[feature_of(a, single, p)];
    mean = f.pooling == MDL_POOL_MEAN;
    return (const TG*)f.grad + ((int64_t)p - f.payload_base) * f.out_stride;
  }

  // Sum of squares of the whole row held by this slot's L lanes.
  __device__ __forceinline__ float row_sumsq(const float (&v)[C]) const {
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < C; ++k) ss += v[k] * v[k];
    const int lane = lane_id();
    for (int m = 1; m < L; m <<= 1) ss += shfl_f(ss, lane ^ m);
    return ss;
  }

  // Finish the run of `key` with summed gradient v: the Adagrad update from
  // the preloaded weight row w and accumulator acc0, or the coalesced row.
  __device__ __forceinline__ void finish(uint32_t key, const float (&v)[C], float ss, float acc0, float (&w)[C],
                                         int64_t uidx) const {
    const int64_t row = (int64_t)key - row_base;
    if (kMode == kModeAdagrad) {
      // scale == 1 leaves every product exact, so unclipped steps are unchanged
      const float acc = acc0 + (ss * (scale * scale)) / (float)dim;
      if (sub == 0) state[row] = acc;
      const float inv = 1.f / (sqrtf(acc) + a.eps);
      if (col_ok) {
#pragma unroll
        for (int k = 0; k < C; ++k) w[k] = w[k] - a.lr * ((v[k] * scale) * inv);
        RowIO<TW, C>::store(W + row * dim + col, w);
      }
    } else if (kMode == kModeCoalesce) {
      const int64_t local = uidx - a.unique_range[2 * t];
      int64_t* rows = (int64_t*)a.rows_addr[t];
      TW* vals = (TW*)a.values_addr[t];
      if (sub == 0) rows[local] = row;
      if (col_ok) RowIO<TW, C>::store(vals + local * dim + col, v);
    }
  }
};

// Keys and payloads of the chunk a wave reduces, staged in LDS: entry i of
// the chunk is s_key[i + 1]; s_key[0] and s_key[len + 1] hold the keys just
// before and after the chunk inside its table (kNone at a table edge).
struct ChunkStage {
  uint32_t key[kChunkMax + 2];
  uint32_t pay[kChunkMax];
};

template <int kMode, bool kOneFeature, typename TW, typename TG, int C>
__device__ __forceinline__ void reduce_chunk_body(const BwdArgs& a, int64_t c, const ChunkRange& r,
                                                  const Reducer<kMode, TW, TG, C>& R, const ChunkStage& st) {
  // Pass groups per iteration: 16 columns of loads in flight per lane.
  constexpr int U = C >= 8 ? 2 : 4;
  constexpr bool adagrad = kMode == kModeAdagrad;
  constexpr bool coalesce = kMode == kModeCoalesce;
  constexpr bool sumsq = kMode == kModeSumsq;
  float ss_acc = 0.f;  // Sumsq: squared norms of the runs this lane's slot finishes
  const int lane = lane_id();
  const uint32_t kNone = 0xffffffffu;
  const int len = (int)(r.c_end - r.c_begin);
  const bool head_open = st.key[0] == st.key[1];
  const bool tail_open = st.key[len + 1] == st.key[len];
  const uint32_t first_key = st.key[1];
  const bool single = head_open && tail_open && first_key == st.key[len];
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  int64_t heads_before = coalesce ? a.head_base[c] : 0;

  float carry[C];
#pragma unroll
  for (int k = 0; k < C; ++k) carry[k] = 0.f;
  uint32_t carry_key = kNone;
  const int G = R.G, L = R.L, slot = R.slot, sub = R.sub;

  for (int base = 0; base < len; base += G * U) {
    float v[U][C], w[U][C], acc0[U], cnt[U];
    uint32_t key[U], pay[U];
    bool fin[U], head[U], own[U], mean[U];
    const TG* gp[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int i = base + u * G + slot;
      const bool valid = i < len;
      const int ii = valid ? i : 0;
      key[u] = valid ? st.key[ii + 1] : kNone;
      pay[u] = st.pay[ii];
      const uint32_t next = st.key[ii + 2];
      fin[u] = valid && next != key[u];
      head[u] = coalesce && valid && st.key[ii] != key[u] &&
                (i > 0 || r.c_begin == r.t_begin || !head_open);
      if (coalesce && valid && i == 0 && r.c_begin == r.t_begin) head[u] = true;
      own[u] = fin[u] && !(head_open && key[u] == first_key);  // the run finishes in this chunk
      if (kOneFeature) {
        mean[u] = R.g_mean;
        gp[u] = valid && R.col_ok ? R.g_base + ((int64_t)pay[u] - R.pbase) * R.g_stride + R.col : zero_row<TG>();
      } else {
        mean[u] = false;
        gp[u] = valid && R.col_ok ? R.grad_row(pay[u], mean[u]) + R.col : zero_row<TG>();
      }
    }
    // Every global load of the group, back to back: gradient rows, bag
    // counts and, for runs that finish here, the weight row and accumulator.
#pragma unroll
    for (int u = 0; u < U; ++u) {
      RowIO<TG, C>::load(gp[u], v[u]);
      cnt[u] = *(mean[u] ? a.bag_count + pay[u] : zero_row<float>());
      if (adagrad) {
        const int64_t row = (int64_t)key[u] - R.row_base;
        RowIO<TW, C>::load(own[u] && R.col_ok ? R.W + row * R.dim + R.col : zero_row<TW>(), w[u]);
        acc0[u] = *(own[u] ? R.state + row : zero_row<float>());
      } else {
#pragma unroll
        for (int k = 0; k < C; ++k) w[u][k] = 0.f;
        acc0[u] = 0.f;
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const float inv = mean[u] ? 1.f / fmaxf(cnt[u], 1.f) : 1.f;
#pragma unroll
      for (int k = 0; k < C; ++k) v[u][k] *= inv;
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      for (int d = 1; d < G; d <<= 1) {
        const int src = slot >= d ? lane - d * L : lane;
        const uint32_t okey = shfl_u(key[u], src);
        float ov[C];
#pragma unroll
        for (int k = 0; k < C; ++k) ov[k] = shfl_f(v[u][k], src);
        if (slot >= d && okey == key[u]) {
#pragma unroll
          for (int k = 0; k < C; ++k) v[u][k] += ov[k];
        }
      }
      if (key[u] == carry_key && key[u] != kNone) {
#pragma unroll
        for (int k = 0; k < C; ++k) v[u][k] += carry[k];
      }
      // Distinct-row index of this entry's run (coalesced layout only).
      int64_t uidx = 0;
      if (coalesce) {
        const uint64_t hm = __ballot(head[u] && sub == 0);
        uidx = heads_before + (int64_t)__popcll(hm & (lt_mask | (1ull << lane))) - 1;
        heads_before += __popcll(hm);
      }
      const float ss = R.row_sumsq(v[u]);
      if (fin[u]) {
        if (!own[u]) {
          if (R.col_ok) {
            float* pf = a.part_first + c * a.max_dim + R.col;
#pragma unroll
            for (int k = 0; k < C; ++k) pf[k] = v[u][k];
          }
        } else if (sumsq) {
          if (sub == 0) ss_acc += ss;
        } else {
          R.finish(key[u], v[u], ss, acc0[u], w[u], uidx);
        }
      }
      const int src = (G - 1) * L + sub;
      const uint32_t lkey = shfl_u(key[u], src);
      const int lfin = shfl_i((int)fin[u], src);
#pragma unroll
      for (int k = 0; k < C; ++k) carry[k] = shfl_f(v[u][k], src);
      carry_key = (lkey != kNone && !lfin) ? lkey : kNone;
    }
  }
  if (tail_open && slot == 0 && R.col_ok) {
    float* pl = a.part_last + c * a.max_dim + R.col;
#pragma unroll
    for (int k = 0; k < C; ++k) pl[k] = carry[k];
  }
  if (sumsq) {
    for (int m = 1; m < kWave; m <<= 1) ss_acc += shfl_f(ss_acc, lane ^ m);
    if (lane == 0) a.chunk_ss[c] = ss_acc;
  }
  if (lane == 0) a.chunk_flags[c] = (head_open ? kHeadOpen : 0) | (tail_open ? kTailOpen : 0) | (single ? kSingle : 0);
}

template <int kMode, typename TW, typename TG, int C>
__device__ __forceinline__ void reduce_chunk(const BwdArgs& a, int64_t c, const ChunkRange& r, ChunkStage& st) {
  Reducer<kMode, TW, TG, C> R(a, r.t);
  if (R.dim > kWave * C) return;  // rejected on the host; never reached
  const int lane = lane_id();
  const uint32_t kNone = 0xffffffffu;
  const int len = (int)(r.c_end - r.c_begin);
  for (int i = lane; i < len; i += kWave) {
    st.key[i + 1] = a.keys[r.c_begin + i];
    st.pay[i] = a.vals[r.c_begin + i];
  }
  if (lane == 0) {
    st.key[0] = r.c_begin > r.t_begin ? a.keys[r.c_begin - 1] : kNone;
    st.key[len + 1] = r.c_end < r.t_end ? a.keys[r.c_end] : kNone;
  }
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
  if (R.single >= 0) reduce_chunk_body<kMode, true, TW, TG, C>(a, c, r, R, st);
  else reduce_chunk_body<kMode, false, TW, TG, C>(a, c, r, R, st);
}

template <int kMode, typename TW, typename TG, int C>
__device__ __forceinline__ void fixup_chunk(const BwdArgs& a, int64_t c, const ChunkRange& r) {
  const int32_t flags = __builtin_amdgcn_readfirstlane(a.chunk_flags[c]);
  if (!(flags & kHeadOpen) || (flags & kSingle)) return;
  Reducer<kMode, TW, TG, C> R(a, r.t);
  if (R.dim > kWave * C) return;  // rejected on the host; never reached
  // Walk back over chunks that lie wholly inside the run to the chunk holding
  // its first entry (never past the table's first chunk).
  const int64_t first_chunk = a.chunk_base[r.t];
  int64_t s = c - 1;
  while (s > first_chunk && (__builtin_amdgcn_readfirstlane(a.chunk_flags[s]) & kSingle)) --s;
  float v[C];
#pragma unroll
  for (int k = 0; k < C; ++k) v[k] = 0.f;
  if (R.col_ok) {
    // Partials of the chunks the run covers, added in chunk order; loads
    // are issued eight chunks at a time.
    int64_t q = s;
    for (; q + 8 <= c; q += 8) {
      float t[8][C];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float* pl = a.part_last + (q + j) * a.max_dim + R.col;
#pragma unroll
        for (int k = 0; k < C; ++k) t[j][k] = pl[k];
      }
#pragma unroll
      for (int j = 0; j < 8; ++j)
#pragma unroll
        for (int k = 0; k < C; ++k) v[k] += t[j][k];
    }
    for (; q < c; ++q) {
      const float* pl = a.part_last + q * a.max_dim + R.col;
#pragma unroll
      for (int k = 0; k < C; ++k) v[k] += pl[k];
    }
    const float* pf = a.part_first + c * a.max_dim + R.col;
#pragma unroll
    for (int k = 0; k < C; ++k) v[k] += pf[k];
  }
  const float ss = R.row_sumsq(v);
  const uint32_t key = a.keys[r.c_begin];
  const int64_t uidx = kMode == kModeCoalesce ? a.head_base[c] - 1 : 0;
  float w[C];
  float acc0 = 0.f;
#pragma unroll
  for (int k = 0; k < C; ++k) w[k] = 0.f;
  if (kMode == kModeAdagrad && R.slot == 0) {
    const int64_t row = (int64_t)key - R.row_base;
    if (R.col_ok) RowIO<TW, C>::load(R.W + row * R.dim + R.col, w);
    acc0 = R.state[row];
  }
  if (kMode == kModeSumsq) {
    // The reduce of chunk c wrote its own runs' share before this launch.
    if (lane_id() == 0) a.chunk_ss[c] += ss;
  } else if (R.slot == 0) {
    R.finish(key, v, ss, acc0, w, uidx);
  }
}

template <bool kFixup, int kMode, typename TW, typename TG, int C>
__global__ __launch_bounds__(kBwdWaves * kWave) void bwd_reduce_kernel(BwdArgs a) {
  const int w = threadIdx.x / kWave;
  // The grid covers the worst-case chunk count; only the first `real` blocks
  // have work.  They are spread round-robin over the XCDs by the hardware, and
  // remapped so that each XCD takes one contiguous range of chunks.
  const int64_t total = uni64b(a.chunk_base[a.T]);
  const int64_t real = (total + kBwdWaves - 1) / kBwdWaves;
  if ((int64_t)blockIdx.x >= real) return;
  const int64_t blk = xcd_block(blockIdx.x, real);
  const int64_t c = uni64b(blk * kBwdWaves + w);
  if (c >= total) return;
  ChunkRange r;
  if (!find_chunk(c, a.T, a.chunk_base, a.table_start, a.table_end, a.table_cb, &r)) return;
  const mdl_table& tb = a.tables[r.t];
  const int cls = row_class(__builtin_amdgcn_readfirstlane(tb.wdtype), __builtin_amdgcn_readfirstlane(tb.gdtype),
                            table_vec(tb));
  if (cls != ClassOf<TW, TG, C>::value) return;  // another class's launch owns it
  if (kFixup) {
    fixup_chunk<kMode, TW, TG, C>(a, c, r);
  } else {
    __shared__ ChunkStage stage[kBwdWaves];
    reduce_chunk<kMode, TW, TG, C>(a, c, r, stage[w]);
  }
}

// ------------------------------------------------------------ host side --

static int validate_tables(const char* who, int32_t T, int32_t max_dim, int64_t n) {
  if (T <= 0) return fail(MDL_ERR_INVALID, std::string(who) + ": need at least one table");
  if (max_dim <= 0) return fail(MDL_ERR_INVALID, std::string(who) + ": max_dim must be positive");
  if (n < 0 || n > 0xffffffffll) return fail(MDL_ERR_UNSUPPORTED, std::string(who) + ": n outside [0, 2^32)");
  return MDL_OK;
}

static int prepare(const mdl_table* tables, int32_t T, int32_t max_dim, uint32_t* keys, uint32_t* payload,
                   int64_t n, int32_t key_bits, void* ws, size_t ws_bytes, hipStream_t s, BwdWs* w,
                   const uint32_t** sk, const uint32_t** sv) {
  const size_t need = carve(w, ws, n, T, max_dim);
  if (ws_bytes < need) return fail(MDL_ERR_WORKSPACE, "backward: workspace too small");
  int in_alt = 0;
  int rc = sort_pairs(keys, payload, w->keys_alt, w->vals_alt, n, key_bits, w->sort_ws, w->sort_bytes, &in_alt, s);
  if (rc) return rc;
  *sk = in_alt ? w->keys_alt : keys;
  *sv = in_alt ? w->vals_alt : payload;
  hipLaunchKernelGGL(bwd_plan_kernel, dim3(1), dim3(kPlanThreads), 0, s, tables, T, *sk, n, w->table_start,
                     w->table_end, w->chunk_base, w->table_cb);
  MDL_CHECK_LAUNCH("bwd_plan_kernel");
  return MDL_OK;
}

static void fill_args(BwdArgs* a, const mdl_feature* feats, int32_t F, const mdl_table* tables, int32_t T,
                      int32_t max_dim, const uint32_t* sk, const uint32_t* sv, const float* bag_count,
                      const BwdWs& w, int64_t n) {
  a->feats = feats;
  a->F = F;
  a->tables = tables;
  a->T = T;
  a->keys = sk;
  a->vals = sv;
  a->bag_count = bag_count;
  a->table_start = w.table_start;
  a->table_end = w.table_end;
  a->chunk_base = w.chunk_base;
  a->table_cb = w.table_cb;
  a->chunk_flags = w.chunk_flags;
  a->head_base = w.head_base;
  a->part_first = w.part_first;
  a->part_last = w.part_last;
  a->chunk_ss = w.chunk_ss;
  a->grad_scale = nullptr;
  a->max_chunks = max_chunks_for(n, T);
  a->max_dim = max_dim;
  a->lr = 0.f;
  a->eps = 0.f;
  a->mode = kModeAdagrad;
  a->rows_addr = nullptr;
  a->values_addr = nullptr;
  a->unique_range = nullptr;
}

template <bool kFixup, typename TW, typename TG, int C>
static int launch_reduce(const BwdArgs& a, uint32_t classes, hipStream_t s) {
  if (classes != 0 && !(classes & (1u << ClassOf<TW, TG, C>::value))) return MDL_OK;
  const int64_t blocks = (a.max_chunks + kBwdWaves - 1) / kBwdWaves;
  if (a.mode == kModeAdagrad)
    hipLaunchKernelGGL((bwd_reduce_kernel<kFixup, kModeAdagrad, TW, TG, C>), dim3((unsigned)blocks),
                       dim3(kBwdWaves * kWave), 0, s, a);
  else if (a.mode == kModeCoalesce)
    hipLaunchKernelGGL((bwd_reduce_kernel<kFixup, kModeCoalesce, TW, TG, C>), dim3((unsigned)blocks),
                       dim3(kBwdWaves * kWave), 0, s, a);
  else
    hipLaunchKernelGGL((bwd_reduce_kernel<kFixup, kModeSumsq, TW, TG, C>), dim3((unsigned)blocks),
                       dim3(kBwdWaves * kWave), 0, s, a);
  MDL_CHECK_LAUNCH(kFixup ? "bwd_fixup_kernel" : "bwd_reduce_kernel");
  return MDL_OK;
}

template <bool kFixup>
static int launch_all(const BwdArgs& a, uint32_t classes, hipStream_t s) {
  int rc = launch_reduce<kFixup, float, float, 4>(a, classes, s);
  if (!rc) rc = launch_reduce<kFixup, float, float, 1>(a, classes, s);
  if (!rc) rc = launch_reduce<kFixup, bf16_t, bf16_t, 8>(a, classes, s);
  if (!rc) rc = launch_reduce<kFixup, bf16_t, bf16_t, 1>(a, classes, s);
  if (!rc) rc = launch_reduce<kFixup, bf16_t, float, 8>(a, classes, s);
  if (!rc) rc = launch_reduce<kFixup, bf16_t, float, 1>(a, classes, s);
  return rc;
}

// Every reduce launch (all classes) before any fix-up launch: a fix-up reads
// partials that the reduce of the same table wrote.
static int run_reduce(const BwdArgs& a, uint32_t classes, hipStream_t s) {
  int rc = launch_all<false>(a, classes, s);
  if (!rc) rc = launch_all<true>(a, classes, s);
  return rc;
}

}  // namespace mdl

using namespace mdl;

extern "C" {

int mdl_sparse_keys(const int64_t* ids, int64_t n, int64_t num_rows, int64_t row_base, int64_t payload_base,
                    int64_t padding_idx, uint32_t* keys, uint32_t* payload, uint32_t sentinel, int32_t* error_count,
                    void* stream) {
  if (n < 0 || n > 0xffffffffll) return fail(MDL_ERR_INVALID, "mdl_sparse_keys: n outside [0, 2^32)");
  if (n == 0) return MDL_OK;
  int64_t blocks = (n + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL(sparse_keys_kernel, dim3((unsigned)blocks), dim3(256), 0, as_stream(stream), ids, n, num_rows,
                     row_base, payload_base, padding_idx, keys, payload, sentinel, error_count);
  MDL_CHECK_LAUNCH("sparse_keys_kernel");
  return MDL_OK;
}

uint32_t mdl_table_classes(const mdl_table* tables, int32_t num_tables) {
  uint32_t m = 0;
  for (int32_t i = 0; i < num_tables; ++i) {
    const mdl_table& t = tables[i];
    m |= 1u << row_class(t.wdtype, t.gdtype, table_vec_of(t.weight, t.dim, t.wdtype));
  }
  return m;
}

size_t mdl_backward_workspace_bytes(int64_t n, int32_t num_tables, int32_t max_dim) {
  BwdWs w;
  // Carving from a null base only measures.
  size_t bytes = carve(&w, nullptr, n, num_tables > 0 ? num_tables : 1, max_dim > 0 ? max_dim : 1);
  // Per-chunk head counts for the coalesced layout (scanned into head_base).
  bytes += ((size_t)(max_chunks_for(n, num_tables > 0 ? num_tables : 1)) * 8 + 255) & ~size_t(255);
  return bytes + 256;
}

int mdl_backward_sort(const mdl_table* tables, int32_t num_tables, int32_t max_dim, uint32_t* sort_keys,
                      uint32_t* sort_payload, int64_t n, int32_t key_bits, void* workspace, size_t workspace_bytes,
                      void* stream) {
  int rc = validate_tables("mdl_backward_sort", num_tables, max_dim, n);
  if (rc) return rc;
  if (n == 0) return MDL_OK;
  BwdWs w;
  const uint32_t *sk, *sv;
  return prepare(tables, num_tables, max_dim, sort_keys, sort_payload, n, key_bits, workspace, workspace_bytes,
                 as_stream(stream), &w, &sk, &sv);
}

// Arguments of the calls that follow mdl_backward_sort: the sorted pairs are
// where the sort's pass count left them.
static int sorted_args(const char* who, BwdArgs* a, const mdl_feature* feats, int32_t num_features,
                       const mdl_table* tables, int32_t num_tables, int32_t max_dim, uint32_t* sort_keys,
                       uint32_t* sort_payload, int64_t n, int32_t key_bits, const float* bag_count,
                       void* workspace, size_t workspace_bytes) {
  BwdWs w;
  const size_t need = carve(&w, workspace, n, num_tables, max_dim);
  if (workspace_bytes < need) return fail(MDL_ERR_WORKSPACE, std::string(who) + ": workspace too small");
  const int passes = (key_bits + 7) / 8;
  const uint32_t* sk = (passes & 1) ? w.keys_alt : sort_keys;
  const uint32_t* sv = (passes & 1) ? w.vals_alt : sort_payload;
  fill_args(a, feats, num_features, tables, num_tables, max_dim, sk, sv, bag_count, w, n);
  return MDL_OK;
}

int mdl_backward_apply(const mdl_feature* feats, int32_t num_features, const mdl_table* tables,
                       int32_t num_tables, int32_t max_dim, uint32_t* sort_keys, uint32_t* sort_payload,
                       int64_t n, int32_t key_bits, const float* bag_count, float lr, float eps,
                       const float* grad_scale, void* workspace, size_t workspace_bytes, uint32_t classes,
                       void* stream) {
  int rc = validate_tables("mdl_backward_apply", num_tables, max_dim, n);
  if (rc) return rc;
  if (n == 0) return MDL_OK;
  BwdArgs a;
  rc = sorted_args("mdl_backward_apply", &a, feats, num_features, tables, num_tables, max_dim, sort_keys,
                   sort_payload, n, key_bits, bag_count, workspace, workspace_bytes);
  if (rc) return rc;
  a.lr = lr;
  a.eps = eps;
  a.grad_scale = grad_scale;
  a.mode = kModeAdagrad;
  return run_reduce(a, classes, as_stream(stream));
}

int mdl_backward_sumsq(const mdl_feature* feats, int32_t num_features, const mdl_table* tables,
                       int32_t num_tables, int32_t max_dim, uint32_t* sort_keys, uint32_t* sort_payload,
                       int64_t n, int32_t key_bits, const float* bag_count, float* sumsq, void* workspace,
                       size_t workspace_bytes, uint32_t classes, void* stream) {
  int rc = validate_tables("mdl_backward_sumsq", num_tables, max_dim, n);
  if (rc) return rc;
  if (!sumsq) return fail(MDL_ERR_INVALID, "mdl_backward_sumsq: null output");
  hipStream_t s = as_stream(stream);
  if (n == 0) return launch_sum_partials(nullptr, 0, nullptr, sumsq, s);
  BwdArgs a;
  rc = sorted_args("mdl_backward_sumsq", &a, feats, num_features, tables, num_tables, max_dim, sort_keys,
                   sort_payload, n, key_bits, bag_count, workspace, workspace_bytes);
  if (rc) return rc;
  a.mode = kModeSumsq;
  rc = run_reduce(a, classes, s);
  if (rc) return rc;
  // chunk_base[T] chunks were reduced; their partials are added in chunk order.
  return launch_sum_partials(a.chunk_ss, 0, a.chunk_base + num_tables, sumsq, s);
}

int mdl_backward_adagrad(const mdl_feature* feats, int32_t num_features, const mdl_table* tables,
                         int32_t num_tables, int32_t max_dim, uint32_t* sort_keys, uint32_t* sort_payload,
                         int64_t n, int32_t key_bits, const float* bag_count, float lr, float eps,
                         const float* grad_scale, void* workspace, size_t workspace_bytes, uint32_t classes,
                         void* stream) {
  int rc = mdl_backward_sort(tables, num_tables, max_dim, sort_keys, sort_payload, n, key_bits, workspace,
                             workspace_bytes, stream);
  if (rc) return rc;
  return mdl_backward_apply(feats, num_features, tables, num_tables, max_dim, sort_keys, sort_payload, n,
                            key_bits, bag_count, lr, eps, grad_scale, workspace, workspace_bytes, classes, stream);
}

int mdl_backward_count(const mdl_table* tables, int32_t num_tables, int32_t max_dim, uint32_t* sort_keys,
                       uint32_t* sort_payload, int64_t n, int32_t key_bits, int64_t* unique_range,
                       void* workspace, size_t workspace_bytes, void* stream) {
  int rc = validate_tables("mdl_backward_count", num_tables, max_dim, n);
  if (rc) return rc;
  hipStream_t s = as_stream(stream);
  BwdWs w;
  const uint32_t *sk, *sv;
  if (n == 0) {
    hipLaunchKernelGGL(unique_range_zero, dim3(1), dim3(256), 0, s, num_tables, unique_range);
    MDL_CHECK_LAUNCH("unique_range_zero");
    return MDL_OK;
  }
  rc = prepare(tables, num_tables, max_dim, sort_keys, sort_payload, n, key_bits, workspace, workspace_bytes, s,
               &w, &sk, &sv);
  if (rc) return rc;
  const int64_t mc = max_chunks_for(n, num_tables);
  int64_t* heads = (int64_t*)((char*)workspace + carve(&w, workspace, n, num_tables, max_dim));
  hipLaunchKernelGGL(count_heads_kernel, dim3((unsigned)((mc + 3) / 4)), dim3(256), 0, s, num_tables,
                     w.chunk_base, w.table_start, w.table_end, w.table_cb, sk, mc, heads);
  MDL_CHECK_LAUNCH("count_heads_kernel");
  rc = mdl_lengths_to_offsets(heads, mc, w.head_base, w.scan_ws, w.scan_bytes, stream);
  if (rc) return rc;
  hipLaunchKernelGGL(unique_range_kernel, dim3((unsigned)((num_tables + 255) / 256)), dim3(256), 0, s,
                     num_tables, w.chunk_base, w.head_base, unique_range);
  MDL_CHECK_LAUNCH("unique_range_kernel");
  return MDL_OK;
}

int mdl_backward_coalesce(const mdl_feature* feats, int32_t num_features, const mdl_table* tables,
                          int32_t num_tables, int32_t max_dim, uint32_t* sort_keys, uint32_t* sort_payload,
                          int64_t n, int32_t key_bits, const float* bag_count, const int64_t* unique_range,
                          const uint64_t* rows_addr, const uint64_t* values_addr, void* workspace,
                          size_t workspace_bytes, uint32_t classes, void* stream) {
  int rc = validate_tables("mdl_backward_coalesce", num_tables, max_dim, n);
  if (rc) return rc;
  if (n == 0) return MDL_OK;
  hipStream_t s = as_stream(stream);
  BwdArgs a;
  rc = sorted_args("mdl_backward_coalesce", &a, feats, num_features, tables, num_tables, max_dim, sort_keys,
                   sort_payload, n, key_bits, bag_count, workspace, workspace_bytes);
  if (rc) return rc;
  a.mode = kModeCoalesce;
  a.rows_addr = rows_addr;
  a.values_addr = values_addr;
  a.unique_range = unique_range;
  return run_reduce(a, classes, s);
}

}  // extern "C"
