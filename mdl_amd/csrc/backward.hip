// Backward of the grouped lookup: sort, unique and deterministic segment
// reduction of per-id gradients, fused with the row-wise Adagrad update (or
// writing a coalesced sparse gradient, or only its squared norm).
//
// After the stable radix sort every distinct (table, row) is one run of equal
// keys whose payloads (gradient rows) appear in input order.  The sorted
// array is cut into chunks of <= kChunkMax entries that never straddle two
// tables, numbered so that the chunks of one kernel variant (row-access
// class x lane width) are contiguous and each table's chunks consecutive.
//
// One wavefront reduces one chunk.  Its G = 64/L lane groups ("slots", L
// lanes per row) each walk a contiguous slice of about kSlotRun (48) entries (fewer in a small call),
// accumulating the per-id gradients in registers: the gradient rows of the
// slice are the only per-entry work, and a run that ends inside the slot that
// began it is finished right there -- its summed gradient goes straight into
// the Adagrad update, with the weight row and accumulator loaded alongside
// the gradient rows (read and written once).  Runs that cross slot bounds are
// joined once per chunk by a segmented scan over the slots' open partials.
// A run that crosses chunk bounds (hot Zipf rows can have 10^4+ entries)
// leaves one fp32 partial per chunk it touches; a second kernel adds those in
// an order fixed by the chunk count and finishes the run.  The summation order depends on the
// chunk layout only, and no floating-point atomics are used, so results do
// not depend on scheduling.
#include <mutex>

#include "common.cuh"

namespace mdl {

int sort_pairs(uint32_t* keys, uint32_t* vals, uint32_t* keys_alt, uint32_t* vals_alt, int64_t n,
               const int64_t* n_dev, int key_bits, void* ws, size_t ws_bytes, int* in_alt, hipStream_t s);
size_t sort_ws_bytes(int64_t n);
int sort_pass_count(int key_bits);
int launch_sum_partials(const float* partial, int64_t m, const int64_t* m_dev, float* out, hipStream_t s);

constexpr int kChunkMax = 512;    // entries of one chunk at most
constexpr int kSlotRun = kPassesPerChunk;  // entries one slot walks in a full chunk
constexpr int kBwdWaves = 4;
constexpr int kBoundThreads = 256;

enum { kHeadOpen = 1, kTailOpen = 2, kSingle = 4 };
// Adagrad: update the rows; Coalesce: write the coalesced gradient; Sumsq:
// only the squared 2-norm of the coalesced gradient (for clipping).
enum { kModeAdagrad = 0, kModeCoalesce = 1, kModeSumsq = 2 };

// One chunk: entries [begin, begin + len) of the sorted array, all of table.
struct ChunkDesc {
  int32_t table;
  int32_t len;
  int64_t begin;
};

struct BwdWs {
  uint32_t* keys_alt;
  uint32_t* vals_alt;
  void* sort_ws;
  size_t sort_bytes;
  int64_t* table_start;   // [T]
  int64_t* table_end;     // [T]
  int64_t* chunk_base;    // [T]   first chunk of table t
  int64_t* num_chunks;    // [1]
  ChunkDesc* desc;        // [max_chunks]
  int32_t* chunk_flags;   // [max_chunks]
  int64_t* head_base;     // [max_chunks+1]
  void* scan_ws;
  size_t scan_bytes;
  float* part_first;      // [max_chunks, max_dim]
  float* part_last;       // [max_chunks, max_dim]
  float* chunk_ss;        // [max_chunks] squared norms of the runs finished per chunk
};

// Entries one slot walks in a full chunk: kSlotRun for a big call; a small
// one takes shorter slices (down to 16) so that its chunks -- one wave each
// -- still give every SIMD a few (about 4096 chunks of 8 slots).
static inline int slot_run_for(int64_t n) {
  const int64_t r = n / 32768;
  return (int)(r < 16 ? 16 : (r > kSlotRun ? kSlotRun : r));
}

// A chunk holds at least slot_run entries unless it is its table's last, so
// a call of n entries has at most ceil(n / slot_run) + T chunks.  That count
// wobbles between 32 K and 34 K chunks while slot_run grows with n; the bound
// below covers it and never decreases with n, so a workspace sized for the
// largest call serves every smaller one.
static inline int64_t max_chunks_for(int64_t n, int32_t T) {
  const int64_t small = 16ll * 32768;
  const int64_t c = n <= small ? (n + 15) / 16 : ((n + 47) / 48 > 34816 ? (n + 47) / 48 : 34816);
  return c + T + 1;
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
  w->chunk_base = (int64_t*)take((size_t)T * 8 + 8);
  w->num_chunks = (int64_t*)take(8);
  w->desc = (ChunkDesc*)take((size_t)mc * sizeof(ChunkDesc));
  w->chunk_flags = (int32_t*)take((size_t)mc * 4);
  w->head_base = (int64_t*)take(((size_t)mc + 1) * 8);
  w->scan_bytes = mdl_offsets_workspace_bytes(mc);
  w->scan_ws = take(w->scan_bytes);
  w->part_first = (float*)take((size_t)mc * max_dim * 4);
  w->part_last = (float*)take((size_t)mc * max_dim * 4);
  w->chunk_ss = (float*)take((size_t)mc * 4);
  return (size_t)(p - start);
}

__device__ __forceinline__ int64_t uni64b(int64_t v) {
  int lo = __builtin_amdgcn_readfirstlane((int)(v & 0xffffffff));
  int hi = __builtin_amdgcn_readfirstlane((int)(v >> 32));
  return (int64_t)(((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo);
}

// ------------------------------------------------------------------ plan --

__device__ __forceinline__ bool table_vec(const mdl_table& tb) {
  return table_vec_of(tb.weight, tb.dim, tb.wdtype);
}

__device__ __forceinline__ int table_variant(const mdl_table& tb) {
  return variant_of(tb.wdtype, tb.gdtype, table_vec(tb), tb.dim);
}

// Entries per chunk of a table: slot_run per slot, one slot per L lanes.
__device__ __forceinline__ int64_t table_chunk_len(const mdl_table& tb, int slot_run) {
  const int c = variant_elems(table_variant(tb));
  const int64_t g = kWave / lanes_for(tb.dim > 0 ? tb.dim : 1, c);
  const int64_t cb = (int64_t)slot_run * g;
  return cb < kChunkMax ? cb : kChunkMax;
}

// Bounds of every table in the sorted keys: block 2t finds the first key >=
// row_base[t], block 2t+1 the first key >= row_base[t] + num_rows.  A k-ary
// search: each round the block probes 256 evenly spaced keys of the
// remaining range, so 2^23 keys take three dependent loads instead of 23.
__global__ __launch_bounds__(kBoundThreads) void bwd_bounds_kernel(const mdl_table* __restrict__ tables,
                                                                   const uint32_t* __restrict__ keys, int64_t n_cap,
                                                                   const int64_t* __restrict__ n_dev,
                                                                   int64_t* table_start, int64_t* table_end) {
  // Sorted entries present: n_cap, or the caller's device count (clamped).
  int64_t n = n_cap;
  if (n_dev != nullptr) {
    const int64_t c = *n_dev;
    n = c < 0 ? 0 : (c > n_cap ? n_cap : c);
  }
  const int32_t t = blockIdx.x >> 1;
  const bool upper = blockIdx.x & 1;
  const uint64_t key = (uint64_t)tables[t].row_base + (upper ? (uint64_t)tables[t].num_rows : 0ull);
  int64_t lo = 0, hi = n;  // the answer lies in [lo, hi]
  const int tid = threadIdx.x;
  while (hi > lo) {
    const int64_t span = hi - lo;
    if (span <= kBoundThreads) {
      const bool less = tid < span && (uint64_t)keys[lo + tid] < key;
      lo += __syncthreads_count(less);
      break;
    }
    // probe p_i = lo + span*(i+1)/(K+1), i < K; keys[p_i] < key holds for a prefix of i
    const int64_t p = lo + span * (tid + 1) / (kBoundThreads + 1);
    const int cnt = __syncthreads_count((uint64_t)keys[p] < key);
    const int64_t nlo = cnt > 0 ? lo + span * cnt / (kBoundThreads + 1) + 1 : lo;
    const int64_t nhi = cnt < kBoundThreads ? lo + span * (cnt + 1) / (kBoundThreads + 1) : hi;
    lo = nlo;
    hi = nhi;
  }
  if (tid == 0) (upper ? table_end : table_start)[t] = lo;
}

// Chunk numbering and descriptors, block t for table t: table t's chunks are
// [chunk_base[t], chunk_base[t] + n_t) in table order -- the block adds up
// the chunk counts of the tables before it -- so neighbouring chunks (one
// XCD's range) share a table; the last block writes the total.  Bounds found
// in keys that are not sorted by table could end before they start or
// overlap: each range is read as [start, max(start, end)) and the chunks
// stop at max_chunks, so every descriptor stays inside the sorted array and
// the workspace.
__global__ __launch_bounds__(256) void bwd_desc_kernel(const mdl_table* __restrict__ tables, int32_t T,
                                                       const int64_t* __restrict__ table_start,
                                                       const int64_t* __restrict__ table_end,
                                                       int64_t* __restrict__ chunk_base,
                                                       int64_t* __restrict__ total,
                                                       ChunkDesc* __restrict__ desc, int64_t max_chunks,
                                                       int slot_run) {
  __shared__ int64_t s_part[256 / kWave];
  const int32_t t = blockIdx.x;
  const int lane = lane_id(), w = threadIdx.x / kWave;
  int64_t before = 0;
  for (int32_t q = threadIdx.x; q < t; q += blockDim.x) {
    const int64_t cq = table_chunk_len(tables[q], slot_run);
    const int64_t sq = table_start[q], eq = table_end[q];
    before += ((eq > sq ? eq : sq) - sq + cq - 1) / cq;
  }
  for (int m = 1; m < kWave; m <<= 1) {
    const int lo = shfl_i((int)(before & 0xffffffff), lane ^ m);
    const int hi = shfl_i((int)(before >> 32), lane ^ m);
    before += (int64_t)(((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo);
  }
  if (lane == 0) s_part[w] = before;
  __syncthreads();
  int64_t base = 0;
  for (int q = 0; q < 256 / kWave; ++q) base += s_part[q];
  const int64_t lo = table_start[t], hi_raw = table_end[t];
  const int64_t hi = hi_raw > lo ? hi_raw : lo;
  const int64_t cb = table_chunk_len(tables[t], slot_run);
  const int64_t room = max_chunks - base;
  const int64_t nch_all = (hi - lo + cb - 1) / cb;
  const int64_t nch = nch_all < room ? nch_all : (room > 0 ? room : 0);
  if (threadIdx.x == 0) {
    chunk_base[t] = base < max_chunks ? base : max_chunks;
    if (t == T - 1) *total = base + nch < max_chunks ? base + nch : max_chunks;
  }
  for (int64_t j = threadIdx.x; j < nch; j += blockDim.x) {
    const int64_t b = lo + j * cb;
    ChunkDesc d;
    d.table = t;
    d.len = (int32_t)(hi - b < cb ? hi - b : cb);
    d.begin = b;
    desc[base + j] = d;
  }
}

// Heads (first entry of a run) per chunk, for the coalesced layout.
__global__ __launch_bounds__(256) void count_heads_kernel(const int64_t* __restrict__ num_chunks,
                                                          const ChunkDesc* __restrict__ desc,
                                                          const int64_t* __restrict__ table_start,
                                                          const uint32_t* __restrict__ keys, int64_t max_chunks,
                                                          int64_t* __restrict__ heads) {
  const int w = threadIdx.x / kWave, lane = lane_id();
  const int64_t c = uni64b((int64_t)blockIdx.x * 4 + w);
  if (c >= max_chunks) return;
  if (c >= *num_chunks) {
    if (lane == 0) heads[c] = 0;
    return;
  }
  const ChunkDesc d = desc[c];
  const int64_t t_begin = table_start[d.table];
  int cnt = 0;
  for (int64_t e = d.begin + lane; e < d.begin + d.len; e += kWave)
    cnt += (e == t_begin || keys[e] != keys[e - 1]) ? 1 : 0;
  for (int m = 1; m < kWave; m <<= 1) cnt += __shfl_xor(cnt, m);
  if (lane == 0) heads[c] = cnt;
}

__global__ void unique_range_end_kernel(int32_t T, const int64_t* table_start, const int64_t* table_end,
                                        const int64_t* chunk_base, const int64_t* head_base,
                                        const mdl_table* __restrict__ tables, int64_t* unique_range,
                                        int slot_run) {
  for (int32_t t = blockIdx.x * blockDim.x + threadIdx.x; t < T; t += gridDim.x * blockDim.x) {
    const int64_t lo = table_start[t], hi = table_end[t];
    const int64_t cb = table_chunk_len(tables[t], slot_run);
    const int64_t nch = (hi - lo + cb - 1) / cb;
    unique_range[2 * t] = head_base[chunk_base[t]];
    unique_range[2 * t + 1] = head_base[chunk_base[t] + nch];
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
  const int64_t* num_chunks;
  const ChunkDesc* desc;
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
__device__ __forceinline__ int32_t feature_of(const BwdArgs& a, uint32_t p) {
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
  int64_t row_base, num_rows;
  float fdim;
  // fields of the table's only feature (single >= 0)
  const TG* g_base;
  int64_t g_stride, pbase;
  bool g_mean, g_pool_none;
  float scale;

  __device__ Reducer(const BwdArgs& args, int32_t table) : a(args), t(table) {
    const mdl_table& tb = a.tables[t];
    dim = __builtin_amdgcn_readfirstlane(tb.dim);
    single = __builtin_amdgcn_readfirstlane(tb.feature);
    W = (TW*)uni64b((int64_t)tb.weight);
    state = (float*)uni64b((int64_t)tb.state);
    row_base = uni64b(tb.row_base);
    num_rows = uni64b(tb.num_rows);
    fdim = (float)dim;
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
    g_pool_none = false;
    scale = 1.f;
    if (kMode == kModeAdagrad && a.grad_scale != nullptr)
      scale = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, *a.grad_scale)));
    if (single >= 0) {
      const mdl_feature& f = a.feats[single];
      g_base = (const TG*)uni64b((int64_t)f.grad);
      g_stride = uni64b(f.out_stride);
      pbase = uni64b(f.payload_base);
      g_mean = __builtin_amdgcn_readfirstlane(f.pooling) == MDL_POOL_MEAN;
      g_pool_none = __builtin_amdgcn_readfirstlane(f.pooling) == MDL_POOL_NONE;
    }
  }

  // Whether a sorted key names a row of this table.  Keys that do not (a
  // caller's key width that does not match its keys leaves them unsorted)
  // touch no weight row or accumulator.
  __device__ __forceinline__ bool row_ok(uint32_t key) const {
    return (uint64_t)((int64_t)key - row_base) < (uint64_t)num_rows;
  }

  // Gradient row of payload p and whether it is divided by its bag count.
  template <bool kOne>
  __device__ __forceinline__ const TG* grad_row(uint32_t p, bool& mean) const {
    if (kOne) {
      mean = g_mean;
      return g_base + ((int64_t)p - pbase) * g_stride;
    }
    const mdl_feature& f = a.feats[feature_of(a, p)];
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
  // the weight row w and accumulator acc0, or the coalesced row at uidx, or
  // (Sumsq) only add its squared norm to ss_acc.
  __device__ __forceinline__ void finish(uint32_t key, const float (&v)[C], float acc0, float (&w)[C], int64_t uidx,
                                         float& ss_acc) const {
    const int64_t row = (int64_t)key - row_base;
    if (kMode == kModeAdagrad) {
      if (!row_ok(key)) return;
      const float ss = row_sumsq(v);
      // The reference update's arithmetic: mean of squares by a true
      // division, eps after the root, the gradient divided by that before the
      // learning-rate product (src/optim.py:53-62).  scale == 1 leaves every
      // product exact, so unclipped steps see the gradient unchanged.
      const float acc = acc0 + (ss * (scale * scale)) / fdim;
      if (sub == 0) st_policy<kUpdatePolicy>(state + row, acc);
      const float den = sqrtf(acc) + a.eps;
      if (col_ok) {
#pragma unroll
        for (int k = 0; k < C; ++k) w[k] = w[k] - a.lr * ((v[k] * scale) / den);
        RowIO<TW, C>::template store<kUpdatePolicy>(W + row * dim + col, w);
      }
    } else if (kMode == kModeCoalesce) {
      const int64_t local = uidx - a.unique_range[2 * t];
      int64_t* rows = (int64_t*)a.rows_addr[t];
      TW* vals = (TW*)a.values_addr[t];
      if (sub == 0) st_policy(rows + local, row);
      if (col_ok) RowIO<TW, C>::template store<kUpdatePolicy>(vals + local * dim + col, v);
    } else {
      const float ss = row_sumsq(v);
      if (sub == 0) ss_acc += ss;
    }
  }
};

// Keys and payloads of the chunk a wave reduces, staged in LDS: entry i of
// the chunk is key[i + 1]; key[0] and key[len + 1] hold the keys just before
// and after the chunk inside its table (kNone at a table edge).  hc[i] counts
// the runs that begin in entries [0, i) (coalesced layout only).
struct ChunkStage {
  uint32_t key[kChunkMax + 2];
  uint32_t pay[kChunkMax];
  uint16_t hc[kChunkMax + 1];
};

template <int C>
__device__ __forceinline__ void zero(float (&v)[C]) {
#pragma unroll
  for (int k = 0; k < C; ++k) v[k] = 0.f;
}

template <int kMode, bool kOne, typename TW, typename TG, int C>
__device__ __forceinline__ void reduce_chunk_body(const BwdArgs& a, int64_t c, const ChunkDesc& d,
                                                  const Reducer<kMode, TW, TG, C>& R, const ChunkStage& st) {
  // Entries per slot per iteration: about MDL_ELEMS_IN_FLIGHT row elements of
  // loads in flight per lane (bf16 weight rows: MDL_BF16_ELEMS_IN_FLIGHT).
  constexpr int U = sizeof(TW) == 2 ? unroll_for<C, MDL_BF16_ELEMS_IN_FLIGHT>() : unroll_for<C>();
  constexpr bool adagrad = kMode == kModeAdagrad;
  constexpr bool coalesce = kMode == kModeCoalesce;
  const uint32_t kNone = 0xffffffffu;
  const int lane = lane_id();
  const int len = d.len;
  const int G = R.G, L = R.L, slot = R.slot;
  const bool head_open = st.key[0] == st.key[1];
  const bool tail_open = st.key[len + 1] == st.key[len];
  const int64_t hb = coalesce ? a.head_base[c] : 0;
  // Gradient rows read once (a table read by one unpooled feature: each
  // output row has one id) can stream past L2, leaving it to rows that are
  // read again (the bag rows of pooled features, read once per id).
  const bool stream_grad = MDL_STREAM_GRAD == 2 || (MDL_STREAM_GRAD == 1 && kOne && R.g_pool_none);
  // This slot's slice [s0, s1) of the chunk.
  // Slices of an odd length start on distinct LDS banks.
  const int K = ((len + G - 1) / G) | 1;
  const int s0 = slot * K;
  const int s1 = s0 + K < len ? s0 + K : len;
  // The slice continues a run that began before it.
  const bool cont = s0 < len && st.key[s0] == st.key[s0 + 1];

  float acc[C], hp[C];
  zero(acc);
  zero(hp);
  float ss_acc = 0.f;
  int hend = -1;      // entry where this slot's first run ends, when that run began before the slice
  bool ended = false;  // a run ended inside the slice

  for (int j = s0; j < s1; j += U) {
    float v[U][C], w[U][C], acc0[U], cnt[U];
    uint32_t key[U];
    bool fin[U], own[U], mean[U], valid[U];
    const TG* gp[U];
    bool e = ended;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int i = j + u;
      valid[u] = i < s1;
      const int ii = valid[u] ? i : s0;
      key[u] = st.key[ii + 1];
      const uint32_t pay = st.pay[ii];
      fin[u] = valid[u] && st.key[ii + 2] != key[u];
      own[u] = fin[u] && (!cont || e);  // the run began inside the slice
      e = e || fin[u];
      mean[u] = false;
      gp[u] = valid[u] && R.col_ok ? R.template grad_row<kOne>(pay, mean[u]) + R.col : zero_row<TG>();
      // The bag count loads without a branch (lanes that need none read the
      // zero row); a table read by one feature decides for the whole wave.
      if (kOne) {
        cnt[u] = R.g_mean ? ld_policy(mean[u] ? a.bag_count + pay : zero_row<float>()) : 0.f;
      } else {
        cnt[u] = ld_policy(mean[u] ? a.bag_count + pay : zero_row<float>());
      }
    }
    // Every global load of the group, back to back: gradient rows and, for
    // runs that finish here, the weight row and accumulator.
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (stream_grad) RowIO<TG, C>::template load<kStream>(gp[u], v[u]);
      else RowIO<TG, C>::load(gp[u], v[u]);
      if (adagrad) {
        const int64_t row = (int64_t)key[u] - R.row_base;
        const bool ld = own[u] && R.row_ok(key[u]);
        RowIO<TW, C>::template load<kUpdatePolicy>(ld && R.col_ok ? R.W + row * R.dim + R.col : zero_row<TW>(), w[u]);
        acc0[u] = ld_policy<kUpdatePolicy>(ld ? R.state + row : zero_row<float>());
      } else {
        zero(w[u]);
        acc0[u] = 0.f;
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      // (an entry past the slice adds its zero row and finishes nothing)
      // grad / max(count, 1) rounded once, then added: the reference's
      // division (src/model.py:570) and its autograd
      const BagDivisor div(mean[u] ? fmaxf(cnt[u], 1.f) : 1.f);
#pragma unroll
      for (int k = 0; k < C; ++k) acc[k] += div(v[u][k]);
      if (fin[u]) {
        if (own[u]) {
          R.finish(key[u], acc, acc0[u], w[u], coalesce ? hb + (int64_t)st.hc[j + u + 1] - 1 : 0, ss_acc);
        } else {
#pragma unroll
          for (int k = 0; k < C; ++k) hp[k] = acc[k];
          hend = j + u;
        }
        zero(acc);
      }
    }
    ended = e;
  }

  // Join the runs that cross slot bounds.  Slot s exports o = the partial of
  // the run open at its end; a slice inside one run (cont, no end) passes the
  // previous slot's export through: o[s] = acc[s] + pass[s] * o[s-1].  The
  // inclusive scan also tells whether that run began before the chunk.
  float o[C];
#pragma unroll
  for (int k = 0; k < C; ++k) o[k] = acc[k];
  bool pass = s0 < len && cont && !ended;
  for (int dd = 1; dd < G; dd <<= 1) {
    const int src = slot >= dd ? lane - dd * L : lane;
    const int opass = shfl_i((int)pass, src);
    float ov[C];
#pragma unroll
    for (int k = 0; k < C; ++k) ov[k] = shfl_f(o[k], src);
    if (slot >= dd) {
      if (pass) {
#pragma unroll
        for (int k = 0; k < C; ++k) o[k] += ov[k];
      }
      pass = pass && opass;
    }
  }
  // The previous slot's export (the part of this slot's first run before it).
  float in[C];
  const int prev = slot > 0 ? lane - L : lane;
#pragma unroll
  for (int k = 0; k < C; ++k) in[k] = shfl_f(o[k], prev);
  // (Every lane takes part in the permute: a source lane outside EXEC reads as 0.)
  const int prev_pass = shfl_i((int)pass, prev);
  const bool in_from_head = slot > 0 ? prev_pass != 0 : head_open;
  if (slot == 0) zero(in);

  if (hend >= 0) {
    // The first run of a continuing slice ends inside it.
    float tot[C];
#pragma unroll
    for (int k = 0; k < C; ++k) tot[k] = in[k] + hp[k];
    if (in_from_head) {
      // it began in an earlier chunk: the fix-up kernel finishes it
      if (R.col_ok) {
        float* pf = a.part_first + c * a.max_dim + R.col;
#pragma unroll
        for (int k = 0; k < C; ++k) pf[k] = tot[k];
      }
    } else {
      const uint32_t key = st.key[hend + 1];
      const int64_t row = (int64_t)key - R.row_base;
      float w[C];
      float acc0 = 0.f;
      zero(w);
      if (adagrad && R.row_ok(key)) {
        if (R.col_ok) RowIO<TW, C>::template load<kUpdatePolicy>(R.W + row * R.dim + R.col, w);
        acc0 = ld_policy<kUpdatePolicy>(R.state + row);
      }
      R.finish(key, tot, acc0, w, coalesce ? hb + (int64_t)st.hc[hend + 1] - 1 : 0, ss_acc);
    }
  }
  // The run open at the chunk's end continues in the next chunk.
  const int last = (len - 1) / K;
  if (tail_open && slot == last && R.col_ok) {
    float* pl = a.part_last + c * a.max_dim + R.col;
#pragma unroll
    for (int k = 0; k < C; ++k) pl[k] = o[k];
  }
  if (kMode == kModeSumsq) {
    for (int m = 1; m < kWave; m <<= 1) ss_acc += shfl_f(ss_acc, lane ^ m);
    if (lane == 0) a.chunk_ss[c] = ss_acc;
  }
  const bool single = head_open && tail_open && st.key[1] == st.key[len];
  (void)kNone;
  if (lane == 0) a.chunk_flags[c] = (head_open ? kHeadOpen : 0) | (tail_open ? kTailOpen : 0) | (single ? kSingle : 0);
}


// The row-wise Adagrad update of a wide row (dim > 64 * C) whose summed
// gradient has squared norm ss: the accumulator first, then each column block
// of the row from grad(b, v), which yields block b of the summed gradient.
// The arithmetic is Reducer::finish's.
template <int kMode, typename TW, typename TG, int C, typename GradOf>
__device__ __forceinline__ void wide_update(const Reducer<kMode, TW, TG, C>& R, uint32_t key, float ss,
                                            GradOf&& grad) {
  constexpr int kSpan = kWave * C;
  const BwdArgs& a = R.a;
  const int lane = lane_id();
  const int64_t row = (int64_t)key - R.row_base;
  const float acc = ld_policy<kUpdatePolicy>(R.state + row) + (ss * (R.scale * R.scale)) / R.fdim;
  if (lane == 0) st_policy<kUpdatePolicy>(R.state + row, acc);
  const float den = sqrtf(acc) + a.eps;
  const int nblk = (R.dim + kSpan - 1) / kSpan;
  for (int b = 0; b < nblk; ++b) {
    float v[C];
    grad(b, v);
    const int col = b * kSpan + lane * C;
    if (col < R.dim) {
      float w[C];
      RowIO<TW, C>::template load<kUpdatePolicy>(R.W + row * R.dim + col, w);
#pragma unroll
      for (int k = 0; k < C; ++k) w[k] = w[k] - a.lr * ((v[k] * R.scale) / den);
      RowIO<TW, C>::template store<kUpdatePolicy>(R.W + row * R.dim + col, w);
    }
  }
}

// Rows wider than the wave's lanes cover at once (dim > 64 * C): the wave
// takes the chunk's runs one at a time and walks each row in column blocks of
// 64 * C elements, reading a run's gradient rows once per block -- twice for
// the update, whose step needs the squared norm of the whole row before any
// element changes (as adagrad_wide_rows does).  Runs cross chunks as in the
// main path: a run that began in an earlier chunk and ends here leaves its
// part in part_first, the run open at the chunk's end in part_last, for the
// fix-up.  Entries of a run add up in their sorted order (deterministic).
// Wide rows are rare (the reference's tables are 8-128 wide); this path is
// general rather than fast.
template <int kMode, bool kOne, typename TW, typename TG, int C>
__device__ void reduce_chunk_wide(const BwdArgs& a, int64_t c, const ChunkDesc& d,
                                  const Reducer<kMode, TW, TG, C>& R, const ChunkStage& st) {
  constexpr int kSpan = kWave * C;
  constexpr int kU = 4;  // entries whose gradient rows load together
  const int lane = lane_id();
  const int len = d.len;
  const int nblk = (R.dim + kSpan - 1) / kSpan;
  const bool head_open = st.key[0] == st.key[1];
  const bool tail_open = st.key[len + 1] == st.key[len];
  const bool single = head_open && tail_open && st.key[1] == st.key[len];
  // Sum of entries [i0, i1)'s gradients over this lane's C columns of block b.
  auto run_sum = [&](int i0, int i1, int b, float (&v)[C]) {
    const int col = b * kSpan + lane * C;
    const bool col_ok = col < R.dim;
    zero(v);
    for (int e = i0; e < i1; e += kU) {
      float g[kU][C], den[kU];
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        const bool ok = e + u < i1;
        const uint32_t pay = st.pay[ok ? e + u : i0];
        bool mean = false;
        const TG* gp = R.template grad_row<kOne>(pay, mean);
        RowIO<TG, C>::load(ok && col_ok ? gp + col : zero_row<TG>(), g[u]);
        const float cnt = ld_policy(ok && mean ? a.bag_count + pay : zero_row<float>());
        den[u] = mean ? fmaxf(cnt, 1.f) : 1.f;
      }
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        const BagDivisor div(den[u]);
#pragma unroll
        for (int k = 0; k < C; ++k) v[k] += div(g[u][k]);
      }
    }
  };
  auto to_parts = [&](float* part, int i0, int i1) {
    for (int b = 0; b < nblk; ++b) {
      float v[C];
      run_sum(i0, i1, b, v);
      const int col = b * kSpan + lane * C;
      if (col < R.dim) {
#pragma unroll
        for (int k = 0; k < C; ++k) part[c * a.max_dim + col + k] = v[k];
      }
    }
  };
  const int64_t hb = kMode == kModeCoalesce ? a.head_base[c] : 0;
  float ss_acc = 0.f;
  for (int i = 0; i < len;) {
    const uint32_t key = st.key[i + 1];
    int j = i + 1;
    while (j < len && st.key[j + 1] == key) ++j;  // the run is entries [i, j)
    if (j == len && tail_open) {
      to_parts(a.part_last, i, j);  // continues in the next chunk (the whole chunk when single)
    } else if (i == 0 && head_open) {
      to_parts(a.part_first, i, j);  // began in an earlier chunk: the fix-up finishes it
    } else if (kMode == kModeCoalesce) {
      const int64_t local = hb + (int64_t)st.hc[j] - 1 - a.unique_range[2 * R.t];
      int64_t* rows = (int64_t*)a.rows_addr[R.t];
      TW* vals = (TW*)a.values_addr[R.t];
      if (lane == 0) st_policy(rows + local, (int64_t)key - R.row_base);
      for (int b = 0; b < nblk; ++b) {
        float v[C];
        run_sum(i, j, b, v);
        const int col = b * kSpan + lane * C;
        if (col < R.dim) RowIO<TW, C>::template store<kUpdatePolicy>(vals + local * R.dim + col, v);
      }
    } else {
      float ss = 0.f;
      for (int b = 0; b < nblk; ++b) {
        float v[C];
        run_sum(i, j, b, v);
        ss += R.row_sumsq(v);
      }
      if (kMode == kModeSumsq) {
        ss_acc += ss;
      } else if (R.row_ok(key)) {
        wide_update(R, key, ss, [&](int b, float (&v)[C]) { run_sum(i, j, b, v); });
      }
    }
    i = j;
  }
  if (kMode == kModeSumsq && lane == 0) a.chunk_ss[c] = ss_acc;
  if (lane == 0) a.chunk_flags[c] = (head_open ? kHeadOpen : 0) | (tail_open ? kTailOpen : 0) | (single ? kSingle : 0);
}

template <int kMode, typename TW, typename TG, int C>
__device__ __forceinline__ void reduce_chunk(const BwdArgs& a, int64_t c, const ChunkDesc& d, ChunkStage& st) {
  Reducer<kMode, TW, TG, C> R(a, d.table);
  const int lane = lane_id();
  const uint32_t kNone = 0xffffffffu;
  const int len = d.len;
  const int64_t t_begin = uni64b(a.table_start[d.table]);
  const int64_t t_end = uni64b(a.table_end[d.table]);
  for (int i = lane; i < len; i += kWave) {
    st.key[i + 1] = a.keys[d.begin + i];
    st.pay[i] = a.vals[d.begin + i];
  }
  if (lane == 0) {
    st.key[0] = d.begin > t_begin ? a.keys[d.begin - 1] : kNone;
    st.key[len + 1] = d.begin + len < t_end ? a.keys[d.begin + len] : kNone;
  }
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
  if (kMode == kModeCoalesce) {
    // hc[i]: runs beginning in entries [0, i)
    const uint64_t lt = lane == 0 ? 0ull : (~0ull >> (kWave - lane));
    int run = 0;
    if (lane == 0) st.hc[0] = 0;
    for (int b = 0; b < len; b += kWave) {
      const int i = b + lane;
      const bool head = i < len && st.key[i] != st.key[i + 1];
      const uint64_t m = __ballot(head);
      if (i < len) st.hc[i + 1] = (uint16_t)(run + __popcll(m & (lt | (1ull << lane))));
      run += __popcll(m);
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
  }
  if (R.dim > kWave * C) {
    if (R.single >= 0) reduce_chunk_wide<kMode, true, TW, TG, C>(a, c, d, R, st);
    else reduce_chunk_wide<kMode, false, TW, TG, C>(a, c, d, R, st);
  } else if (R.single >= 0) {
    reduce_chunk_body<kMode, true, TW, TG, C>(a, c, d, R, st);
  } else {
    reduce_chunk_body<kMode, false, TW, TG, C>(a, c, d, R, st);
  }
}


// The fix-up of a wide row (dim > 64 * C): the run's parts, chunk s's to
// chunk c - 1's part_last and chunk c's part_first, added in chunk order per
// column block; the update reads them twice (squared norm, then the step).
template <int kMode, typename TW, typename TG, int C>
__device__ void fixup_chunk_wide(const BwdArgs& a, int64_t c, const ChunkDesc& d,
                                 const Reducer<kMode, TW, TG, C>& R, int64_t s) {
  constexpr int kSpan = kWave * C;
  const int lane = lane_id();
  const int nblk = (R.dim + kSpan - 1) / kSpan;
  auto parts = [&](int b, float (&v)[C]) {
    const int col = b * kSpan + lane * C;
    zero(v);
    if (col < R.dim) {
      for (int64_t q = s; q < c; ++q) {
        const float* pl = a.part_last + q * a.max_dim + col;
#pragma unroll
        for (int k = 0; k < C; ++k) v[k] += pl[k];
      }
      const float* pf = a.part_first + c * a.max_dim + col;
#pragma unroll
      for (int k = 0; k < C; ++k) v[k] += pf[k];
    }
  };
  const uint32_t key = a.keys[d.begin];
  if (kMode == kModeCoalesce) {
    const int64_t local = a.head_base[c] - 1 - a.unique_range[2 * R.t];
    int64_t* rows = (int64_t*)a.rows_addr[R.t];
    TW* vals = (TW*)a.values_addr[R.t];
    if (lane == 0) st_policy(rows + local, (int64_t)key - R.row_base);
    for (int b = 0; b < nblk; ++b) {
      float v[C];
      parts(b, v);
      const int col = b * kSpan + lane * C;
      if (col < R.dim) RowIO<TW, C>::template store<kUpdatePolicy>(vals + local * R.dim + col, v);
    }
    return;
  }
  float ss = 0.f;
  for (int b = 0; b < nblk; ++b) {
    float v[C];
    parts(b, v);
    ss += R.row_sumsq(v);
  }
  if (kMode == kModeSumsq) {
    // The reduce of chunk c wrote its own runs' share before this launch.
    if (lane == 0) a.chunk_ss[c] += ss;
  } else if (R.row_ok(key)) {
    wide_update(R, key, ss, parts);
  }
}

template <int kMode, typename TW, typename TG, int C>
__device__ __forceinline__ void fixup_chunk(const BwdArgs& a, int64_t c, const ChunkDesc& d, int32_t flags) {
  Reducer<kMode, TW, TG, C> R(a, d.table);
  // Walk back over chunks that lie wholly inside the run to the chunk holding
  // its first entry (never past the table's first chunk).
  // The wave reads 64 chunks' flags per step (a Zipf head row spans many
  // chunks; one dependent load per chunk made this walk the fix-up's cost).
  const int64_t first_chunk = uni64b(a.chunk_base[d.table]);
  int64_t s = c - 1;
  for (;;) {
    const int64_t q = s - lane_id();
    const bool inside = q > first_chunk;
    const int32_t fq = a.chunk_flags[inside ? q : first_chunk];
    const uint64_t stop = __ballot(!inside || !(fq & kSingle));
    if (stop) {
      s -= __builtin_ctzll(stop);
      break;
    }
    s -= kWave;
  }
  if (R.dim > kWave * C) {
    fixup_chunk_wide<kMode, TW, TG, C>(a, c, d, R, s);
    return;
  }
  float v[C];
  zero(v);
  // Partials of the chunks the run covers: slot g adds chunks s + g,
  // s + g + G, ... (eight loads in flight per lane), then the G slot sums
  // meet in a butterfly.  Each pairwise add is commutative, so every lane
  // ends with the same bits and the order is fixed from run to run.
  {
    const int G = R.G;
    int64_t q = s + R.slot;
    if (R.col_ok) {
      for (; q + 7 * G < c; q += 8 * G) {
        float tt[8][C];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float* pl = a.part_last + (q + j * G) * a.max_dim + R.col;
#pragma unroll
          for (int k = 0; k < C; ++k) tt[j][k] = pl[k];
        }
#pragma unroll
        for (int j = 0; j < 8; ++j)
#pragma unroll
          for (int k = 0; k < C; ++k) v[k] += tt[j][k];
      }
      for (; q < c; q += G) {
        const float* pl = a.part_last + q * a.max_dim + R.col;
#pragma unroll
        for (int k = 0; k < C; ++k) v[k] += pl[k];
      }
    }
    for (int m = R.L; m < kWave; m <<= 1)
#pragma unroll
      for (int k = 0; k < C; ++k) v[k] += shfl_f(v[k], lane_id() ^ m);
    if (R.col_ok) {
      const float* pf = a.part_first + c * a.max_dim + R.col;
#pragma unroll
      for (int k = 0; k < C; ++k) v[k] += pf[k];
    }
  }
  const uint32_t key = a.keys[d.begin];
  const int64_t uidx = kMode == kModeCoalesce ? a.head_base[c] - 1 : 0;
  float w[C];
  float acc0 = 0.f;
  zero(w);
  if (kMode == kModeAdagrad && R.slot == 0 && R.row_ok(key)) {
    const int64_t row = (int64_t)key - R.row_base;
    if (R.col_ok) RowIO<TW, C>::template load<kUpdatePolicy>(R.W + row * R.dim + R.col, w);
    acc0 = ld_policy<kUpdatePolicy>(R.state + row);
  }
  float ss = 0.f;
  if (R.slot == 0) R.finish(key, v, acc0, w, uidx, ss);
  if (kMode == kModeSumsq) {
    // The reduce of chunk c wrote its own runs' share before this launch.
    if (lane_id() == 0) a.chunk_ss[c] += ss;
  }
  (void)flags;
}

template <bool kFixup, int kMode, typename TW, typename TG, bool kVec>
__global__ MDL_OCCUPANCY __launch_bounds__(kBwdWaves * kWave) void bwd_reduce_kernel(BwdArgs a) {
  const int w = threadIdx.x / kWave;
  // One wave per chunk.  The grid covers the worst-case chunk count; only the
  // first `real` blocks have work (the rest return at once).  The hardware
  // deals blocks round-robin to the XCDs; they are remapped so that each XCD
  // takes one contiguous range of chunks, whose rows and gradient slices then
  // share that XCD's L2.
  const int64_t total = uni64b(*a.num_chunks);
  const int64_t real = (total + kBwdWaves - 1) / kBwdWaves;
  if ((int64_t)blockIdx.x >= real) return;
  const int64_t blk = xcd_block(blockIdx.x, real);
  const int64_t c = uni64b(blk * kBwdWaves + w);
  if (c >= total) return;
  int32_t flags = 0;
  if (kFixup) {
    flags = __builtin_amdgcn_readfirstlane(a.chunk_flags[c]);
    if (!(flags & kHeadOpen) || (flags & kSingle)) return;
  }
  ChunkDesc d;
  d.table = __builtin_amdgcn_readfirstlane(a.desc[c].table);
  d.len = __builtin_amdgcn_readfirstlane(a.desc[c].len);
  d.begin = uni64b(a.desc[c].begin);
  const int v = table_variant(a.tables[d.table]);
  if (v / kWidths != ClassOf<TW, TG, kVec>::value) return;  // another class's launch owns it
  if (kFixup) {
    with_width<TW, kVec>(v % kWidths, [&]<int C>() { fixup_chunk<kMode, TW, TG, C>(a, c, d, flags); });
  } else {
    __shared__ ChunkStage stage[kBwdWaves];
    with_width<TW, kVec>(v % kWidths, [&]<int C>() { reduce_chunk<kMode, TW, TG, C>(a, c, d, stage[w]); });
  }
}

// ------------------------------------------------------------ host side --

static int validate_tables(const char* who, int32_t T, int32_t max_dim, int64_t n) {
  if (T <= 0) return fail(MDL_ERR_INVALID, std::string(who) + ": need at least one table");
  if (max_dim <= 0) return fail(MDL_ERR_INVALID, std::string(who) + ": max_dim must be positive");
  if (n < 0 || n > 0xffffffffll) return fail(MDL_ERR_UNSUPPORTED, std::string(who) + ": n outside [0, 2^32)");
  return MDL_OK;
}

static int validate_classes(const char* who, uint32_t classes) {
  if (classes & MDL_CLASSES_UNSUPPORTED)
    return fail(MDL_ERR_UNSUPPORTED,
                std::string(who) + ": the class mask carries the reserved MDL_CLASSES_UNSUPPORTED bit");
  return MDL_OK;
}

static int plan(const mdl_table* tables, int32_t T, const uint32_t* sk, int64_t n, const int64_t* n_dev,
                const BwdWs& w, hipStream_t s) {
  hipLaunchKernelGGL(bwd_bounds_kernel, dim3((unsigned)(2 * T)), dim3(kBoundThreads), 0, s, tables, sk, n, n_dev,
                     w.table_start, w.table_end);
  MDL_CHECK_LAUNCH("bwd_bounds_kernel");
  hipLaunchKernelGGL(bwd_desc_kernel, dim3((unsigned)T), dim3(256), 0, s, tables, T, w.table_start, w.table_end,
                     w.chunk_base, w.num_chunks, w.desc, max_chunks_for(n, T), slot_run_for(n));
  MDL_CHECK_LAUNCH("bwd_desc_kernel");
  return MDL_OK;
}

static int prepare(const mdl_table* tables, int32_t T, int32_t max_dim, uint32_t* keys, uint32_t* payload,
                   int64_t n, const int64_t* n_dev, int32_t key_bits, void* ws, size_t ws_bytes, hipStream_t s,
                   BwdWs* w, const uint32_t** sk, const uint32_t** sv) {
  const size_t need = carve(w, ws, n, T, max_dim);
  if (ws_bytes < need) return fail(MDL_ERR_WORKSPACE, "backward: workspace too small");
  int in_alt = 0;
  int rc = sort_pairs(keys, payload, w->keys_alt, w->vals_alt, n, n_dev, key_bits, w->sort_ws, w->sort_bytes,
                      &in_alt, s);
  if (rc) return rc;
  *sk = in_alt ? w->keys_alt : keys;
  *sv = in_alt ? w->vals_alt : payload;
  return plan(tables, T, *sk, n, n_dev, *w, s);
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
  a->num_chunks = w.num_chunks;
  a->desc = w.desc;
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

template <bool kFixup>
struct LaunchReduce {
  const BwdArgs& a;
  hipStream_t s;
  int64_t grid_blocks;
  template <typename TW, typename TG, bool kVec>
  int operator()() const {
    const int64_t blocks = grid_blocks;
    if (a.mode == kModeAdagrad)
      hipLaunchKernelGGL((bwd_reduce_kernel<kFixup, kModeAdagrad, TW, TG, kVec>), dim3((unsigned)blocks),
                         dim3(kBwdWaves * kWave), 0, s, a);
    else if (a.mode == kModeCoalesce)
      hipLaunchKernelGGL((bwd_reduce_kernel<kFixup, kModeCoalesce, TW, TG, kVec>), dim3((unsigned)blocks),
                         dim3(kBwdWaves * kWave), 0, s, a);
    else
      hipLaunchKernelGGL((bwd_reduce_kernel<kFixup, kModeSumsq, TW, TG, kVec>), dim3((unsigned)blocks),
                         dim3(kBwdWaves * kWave), 0, s, a);
    MDL_CHECK_LAUNCH(kFixup ? "bwd_fixup_kernel" : "bwd_reduce_kernel");
    return MDL_OK;
  }
};

// Every reduce launch (all classes) before any fix-up launch: a fix-up reads
// partials that the reduce of the same table wrote.
static int run_reduce(const BwdArgs& a, uint32_t variants, hipStream_t s) {
  if (variants & MDL_CLASSES_UNSUPPORTED)
    return fail(MDL_ERR_UNSUPPORTED,
                "backward: the class mask carries the reserved MDL_CLASSES_UNSUPPORTED bit");
  const int64_t blocks = (a.max_chunks + kBwdWaves - 1) / kBwdWaves;
  if (blocks > 0x7fffffffll) return fail(MDL_ERR_UNSUPPORTED, "backward: too many chunks");
  int rc = for_each_class(variants, LaunchReduce<false>{a, s, blocks});
  if (!rc) rc = for_each_class(variants, LaunchReduce<true>{a, s, blocks});
  return rc;
}

// ------------------------------------------------------ capacity padding --
//
// Coalesced gradients sized to a capacity known on the host (a table's id
// count bounds its distinct rows): entries [U_t, cap_t) of table t repeat
// its last row (row 0 when it has none) with zero values, so the whole
// buffer is a valid uncoalesced COO gradient whose sum is the coalesced one.
// Work: units of kPadRows entries over the capacity prefix, one wave each.
constexpr int64_t kPadRows = 64;

__global__ __launch_bounds__(256) void pad_kernel(const mdl_table* __restrict__ tables, int32_t T,
                                                  const int64_t* __restrict__ unique_range,
                                                  const uint64_t* __restrict__ rows_addr,
                                                  const uint64_t* __restrict__ values_addr,
                                                  const int64_t* __restrict__ capacity,
                                                  const int64_t* __restrict__ unit_first, int64_t units) {
  const int64_t unit = (int64_t)blockIdx.x * 4 + threadIdx.x / kWave;
  if (unit >= units) return;
  int lo = 0, hi = T - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (unit_first[mid] <= unit) lo = mid;
    else hi = mid - 1;
  }
  const int t = lo;
  const int64_t u = unique_range[2 * t + 1] - unique_range[2 * t];
  const int64_t r0 = (unit - unit_first[t]) * kPadRows;
  const int64_t cap = capacity[t];
  const int64_t r1 = r0 + kPadRows < cap ? r0 + kPadRows : cap;
  const int64_t b = r0 > u ? r0 : u;
  if (b >= r1 || rows_addr[t] == 0) return;
  int64_t* rows = reinterpret_cast<int64_t*>(rows_addr[t]);
  const int lane = lane_id();
  const int64_t fill = u > 0 ? rows[u - 1] : 0;
  for (int64_t i = b + lane; i < r1; i += kWave) rows[i] = fill;
  const mdl_table& tb = tables[t];
  const int64_t esz = tb.wdtype == MDL_BF16 ? 2 : 4;
  const int64_t bytes = (r1 - b) * (int64_t)tb.dim * esz;
  char* v = reinterpret_cast<char*>(values_addr[t]) + b * (int64_t)tb.dim * esz;
  // 4-byte stores: rows of any dim (a bf16 row of odd dim ends on 2 bytes).
  if (bytes % 4 == 0 && reinterpret_cast<uint64_t>(v) % 4 == 0) {
    uint32_t* w = reinterpret_cast<uint32_t*>(v);
    for (int64_t i = lane; i < bytes / 4; i += kWave) w[i] = 0u;
  } else {
    uint16_t* w = reinterpret_cast<uint16_t*>(v);
    for (int64_t i = lane; i < bytes / 2; i += kWave) w[i] = 0;
  }
}

// --------------------------------------------------- allocation-free call --
//
// Scratch of mdl_backward_adagrad_noalloc: one static device array (each GPU
// the library runs on holds its own copy until the process ends).  Host code
// never passes the array's name to a kernel -- in host code that name is a
// stand-in, not a device address -- but the address hipGetSymbolAddress
// returns for the current device, looked up once per device on its first
// call.
constexpr size_t kNoAllocScratchBytes = size_t(64) << 20;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[kMaxDevices];

// The scratch of the device the call runs on: the current device, which a
// non-null stream must belong to (its kernels run on the stream's device, and
// the array's address differs per device).
static int scratch_for_stream(hipStream_t stream, void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return check_hip(e, "hipGetDevice");
  if (dev < 0 || dev >= kMaxDevices) return fail(MDL_ERR_UNSUPPORTED, "mdl_backward_adagrad_noalloc: device index");
  if (stream != nullptr) {
    hipDevice_t sdev = -1;
    e = hipStreamGetDevice(stream, &sdev);
    if (e != hipSuccess) return check_hip(e, "hipStreamGetDevice");
    if ((int)sdev != dev)
      return fail(MDL_ERR_INVALID, "mdl_backward_adagrad_noalloc: the stream belongs to device " +
                                       std::to_string((int)sdev) + " but device " + std::to_string(dev) +
                                       " is current; make the stream's device current");
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return check_hip(e, "hipGetSymbolAddress(scratch)");
    if (p == nullptr) return fail(MDL_ERR_HIP, "hipGetSymbolAddress(scratch) returned a null address");
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return MDL_OK;
}

}  // namespace mdl

using namespace mdl;

extern "C" {

size_t mdl_noalloc_scratch_bytes(void) { return kNoAllocScratchBytes; }

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
    const int v = variant_of(t.wdtype, t.gdtype, table_vec_of(t.weight, t.dim, t.wdtype), t.dim);
    m |= 1u << v;
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
                      uint32_t* sort_payload, int64_t n, const int64_t* count, int32_t key_bits, void* workspace,
                      size_t workspace_bytes, void* stream) {
  int rc = validate_tables("mdl_backward_sort", num_tables, max_dim, n);
  if (rc) return rc;
  if (n == 0) return MDL_OK;
  BwdWs w;
  const uint32_t *sk, *sv;
  return prepare(tables, num_tables, max_dim, sort_keys, sort_payload, n, count, key_bits, workspace,
                 workspace_bytes, as_stream(stream), &w, &sk, &sv);
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
  const int passes = sort_pass_count(key_bits);
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
  if (!rc) rc = validate_classes("mdl_backward_apply", classes);
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
  if (!rc) rc = validate_classes("mdl_backward_sumsq", classes);
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
  // *num_chunks chunks were reduced; their partials are added in chunk order.
  return launch_sum_partials(a.chunk_ss, 0, a.num_chunks, sumsq, s);
}

int mdl_backward_adagrad(const mdl_feature* feats, int32_t num_features, const mdl_table* tables,
                         int32_t num_tables, int32_t max_dim, uint32_t* sort_keys, uint32_t* sort_payload,
                         int64_t n, const int64_t* count, int32_t key_bits, const float* bag_count, float lr,
                         float eps, const float* grad_scale, void* workspace, size_t workspace_bytes,
                         uint32_t classes, void* stream) {
  int rc = validate_classes("mdl_backward_adagrad", classes);
  if (rc) return rc;
  rc = mdl_backward_sort(tables, num_tables, max_dim, sort_keys, sort_payload, n, count, key_bits, workspace,
                             workspace_bytes, stream);
  if (rc) return rc;
  return mdl_backward_apply(feats, num_features, tables, num_tables, max_dim, sort_keys, sort_payload, n,
                            key_bits, bag_count, lr, eps, grad_scale, workspace, workspace_bytes, classes, stream);
}

int mdl_backward_count(const mdl_table* tables, int32_t num_tables, int32_t max_dim, uint32_t* sort_keys,
                       uint32_t* sort_payload, int64_t n, const int64_t* count, int32_t key_bits,
                       int64_t* unique_range, void* workspace, size_t workspace_bytes, void* stream) {
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
  rc = prepare(tables, num_tables, max_dim, sort_keys, sort_payload, n, count, key_bits, workspace, workspace_bytes,
               s, &w, &sk, &sv);
  if (rc) return rc;
  const int64_t mc = max_chunks_for(n, num_tables);
  int64_t* heads = (int64_t*)((char*)workspace + carve(&w, workspace, n, num_tables, max_dim));
  hipLaunchKernelGGL(count_heads_kernel, dim3((unsigned)((mc + 3) / 4)), dim3(256), 0, s, w.num_chunks, w.desc,
                     w.table_start, sk, mc, heads);
  MDL_CHECK_LAUNCH("count_heads_kernel");
  rc = mdl_lengths_to_offsets(heads, mc, w.head_base, w.scan_ws, w.scan_bytes, stream);
  if (rc) return rc;
  hipLaunchKernelGGL(unique_range_end_kernel, dim3((unsigned)((num_tables + 255) / 256)), dim3(256), 0, s,
                     num_tables, w.table_start, w.table_end, w.chunk_base, w.head_base, tables, unique_range,
                     slot_run_for(n));
  MDL_CHECK_LAUNCH("unique_range_end_kernel");
  return MDL_OK;
}

int mdl_backward_coalesce(const mdl_feature* feats, int32_t num_features, const mdl_table* tables,
                          int32_t num_tables, int32_t max_dim, uint32_t* sort_keys, uint32_t* sort_payload,
                          int64_t n, int32_t key_bits, const float* bag_count, const int64_t* unique_range,
                          const uint64_t* rows_addr, const uint64_t* values_addr, void* workspace,
                          size_t workspace_bytes, uint32_t classes, void* stream) {
  int rc = validate_tables("mdl_backward_coalesce", num_tables, max_dim, n);
  if (!rc) rc = validate_classes("mdl_backward_coalesce", classes);
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

int mdl_backward_adagrad_noalloc(const mdl_feature* feats, int32_t num_features, const mdl_table* tables,
                                 int32_t num_tables, int32_t max_dim, uint32_t* sort_keys, uint32_t* sort_payload,
                                 int64_t n, const int64_t* count, int32_t key_bits, const float* bag_count, float lr,
                                 float eps, const float* grad_scale, uint32_t classes, void* stream) {
  int rc = validate_tables("mdl_backward_adagrad_noalloc", num_tables, max_dim, n);
  if (rc) return rc;
  const size_t need = mdl_backward_workspace_bytes(n, num_tables, max_dim);
  if (need > kNoAllocScratchBytes)
    return fail(MDL_ERR_UNSUPPORTED, "mdl_backward_adagrad_noalloc: this call needs " + std::to_string(need) +
                                         " bytes of scratch; the static scratch holds " +
                                         std::to_string(kNoAllocScratchBytes) +
                                         " (fewer entries, tables or a smaller max_dim fit)");
  void* ws = nullptr;
  rc = scratch_for_stream(as_stream(stream), &ws);
  if (rc) return rc;
  return mdl_backward_adagrad(feats, num_features, tables, num_tables, max_dim, sort_keys, sort_payload, n, count,
                              key_bits, bag_count, lr, eps, grad_scale, ws, kNoAllocScratchBytes, classes, stream);
}

int mdl_backward_pad(const mdl_table* tables, int32_t num_tables, const int64_t* unique_range,
                     const uint64_t* rows_addr, const uint64_t* values_addr, const int64_t* capacity,
                     const int64_t* unit_first, int64_t units, void* stream) {
  if (num_tables <= 0 || units < 0) return fail(MDL_ERR_INVALID, "mdl_backward_pad: bad sizes");
  if (units == 0) return MDL_OK;
  if (!tables || !unique_range || !rows_addr || !values_addr || !capacity || !unit_first)
    return fail(MDL_ERR_INVALID, "mdl_backward_pad: null pointer");
  const int64_t blocks = (units + 3) / 4;
  if (blocks > 0x7fffffffll) return fail(MDL_ERR_UNSUPPORTED, "mdl_backward_pad: too many rows");
  hipLaunchKernelGGL(pad_kernel, dim3((unsigned)blocks), dim3(256), 0, as_stream(stream), tables, num_tables,
                     unique_range, rows_addr, values_addr, capacity, unit_first, units);
  MDL_CHECK_LAUNCH("pad_kernel");
  return MDL_OK;
}

}  // extern "C"
