// Grouped embedding lookup and bag pooling for gfx950.
//
// One wavefront owns one chunk (a run of whole bags of one feature, or a run
// of ids of an unpooled feature).  A row of `dim` elements is spread over L
// lanes of C elements each (C = 4 or 8 fp32, 8 bf16, in 16-byte accesses;
// 1 for rows that are not 16-byte aligned), so a wave holds G = 64 / L rows
// at a time.
//
// Pooling: the chunk's ids form one flat stream in which bags are consecutive
// segments.  The G lane groups ("slots") each walk a contiguous slice of that
// stream, adding rows into registers; a bag that ends inside the slot that
// began it is divided (mean) and written right there, so every id costs a
// row load and C adds whatever the bag lengths (ragged bags of 1..32 ids keep
// all lanes busy).  Bags that cross slot bounds are joined once per chunk by
// a segmented scan over the slots' open partial sums.  The summation order is
// fixed by the chunk layout alone (deterministic).  Bag bounds and the
// table row of every id are staged in LDS once per chunk.
#include "common.cuh"

namespace mdl {

constexpr int kFwdWaves = 4;
constexpr int kMaxBagsPerChunk = 256;

struct FwdArgs {
  const mdl_feature* feats;
  const mdl_chunk* chunks;
  int64_t num_chunks;
  const int64_t* ids;
  int64_t num_ids;  // entries of ids: every feature's id range is clamped into [0, num_ids)
  const int64_t* offsets;
  uint32_t* keys;
  uint32_t* payload;
  const int64_t* key_origin;  // device position that is entry 0 of keys/payload (NULL: 0)
  int64_t key_lo;             // ids before it belong to another call (set per wave)
  float* bag_count;
  int32_t* error_count;
  uint32_t sentinel;
};

// Wave-uniform copy of the descriptor fields a chunk needs.
struct Feat {
  const void* weight;
  void* out;
  int64_t num_rows, out_stride, row_base, payload_base, ids_begin, num_ids, bag_base, num_bags;
  int dim, wdtype, odtype, pooling, flags, padding_idx;
};

__device__ __forceinline__ int64_t uni64(int64_t v) {
  int lo = __builtin_amdgcn_readfirstlane((int)(v & 0xffffffff));
  int hi = __builtin_amdgcn_readfirstlane((int)(v >> 32));
  return (int64_t)(((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo);
}
__device__ __forceinline__ int uni32(int v) { return __builtin_amdgcn_readfirstlane(v); }

__device__ __forceinline__ Feat load_feat(const mdl_feature* p) {
  Feat f;
  f.weight = (const void*)uni64((int64_t)p->weight);
  f.out = (void*)uni64((int64_t)p->out);
  f.num_rows = uni64(p->num_rows);
  f.out_stride = uni64(p->out_stride);
  f.row_base = uni64(p->row_base);
  f.payload_base = uni64(p->payload_base);
  f.ids_begin = uni64(p->ids_begin);
  f.num_ids = uni64(p->num_ids);
  f.bag_base = uni64(p->bag_base);
  f.num_bags = uni64(p->num_bags);
  f.dim = uni32(p->dim);
  f.wdtype = uni32(p->wdtype);
  f.odtype = uni32(p->odtype);
  f.pooling = uni32(p->pooling);
  f.flags = uni32(p->flags);
  f.padding_idx = uni32(p->padding_idx);
  return f;
}

// The feature's id range for this call.  With MDL_FLAG_IDS_FROM_OFFSETS it
// is [offsets[bag_base], offsets[bag_base + nb]) (nb = num_bags, or 1 for an
// unpooled feature's pseudo-bag), so a batch whose bag lengths change needs no
// new descriptors: the offsets scan of its lengths places every feature.  The
// descriptor's [ids_begin, ids_begin + num_ids) is then only a bound.  Either
// way the range is clamped into the call's [0, num_ids), so lengths that do
// not add up give an error count and wrong sums, never an access outside ids.
__device__ __forceinline__ void bind_range(Feat& f, const FwdArgs& a) {
  int64_t lo = f.ids_begin, hi = f.ids_begin + f.num_ids;
  if ((f.flags & MDL_FLAG_IDS_FROM_OFFSETS) && a.offsets != nullptr) {
    const int64_t nb = f.pooling == MDL_POOL_NONE ? 1 : f.num_bags;
    int64_t olo = uni64(a.offsets[f.bag_base]);
    int64_t ohi = uni64(a.offsets[f.bag_base + nb]);
    olo = olo < lo ? lo : (olo > hi ? hi : olo);
    ohi = ohi < olo ? olo : (ohi > hi ? hi : ohi);
    lo = olo;
    hi = ohi;
  }
  lo = lo < a.key_lo ? a.key_lo : (lo > a.num_ids ? a.num_ids : lo);
  hi = hi < lo ? lo : (hi > a.num_ids ? a.num_ids : hi);
  f.ids_begin = lo;
  f.num_ids = hi - lo;
}

__device__ __forceinline__ int feat_variant(const Feat& f) {
  return variant_of(f.wdtype, f.odtype,
                    feature_vec((uint64_t)f.weight, (uint64_t)f.out, f.dim, f.out_stride, f.wdtype, f.odtype),
                    f.dim);
}

__device__ __forceinline__ void wave_sync() { __builtin_amdgcn_wave_barrier(); __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront"); }

template <int C>
__device__ __forceinline__ void zero_c(float (&v)[C]) {
#pragma unroll
  for (int k = 0; k < C; ++k) v[k] = 0.f;
}

// ------------------------------------------------------------ unpooled --

template <typename TW, typename TO, int C>
__device__ __forceinline__ void gather_chunk(const Feat& f, int64_t first, int count, const FwdArgs& a) {
  constexpr int kUnroll = unroll_for<C>();
  const int lane = lane_id();
  const int L = lanes_for(f.dim, C);
  const int G = kWave / L;
  const int slot = lane / L, sub = lane % L;
  const int ncb = (f.dim + L * C - 1) / (L * C);
  const TW* W = static_cast<const TW*>(f.weight);
  TO* out = static_cast<TO*>(f.out);
  const int64_t* ids = a.ids + f.ids_begin + first;
  const int step = G * kUnroll;
  constexpr bool kSplit = MDL_SPLIT_ROWS && std::is_same_v<TW, float> && std::is_same_v<TO, float> && C == 8;
  for (int cb = 0; cb < ncb; ++cb) {
    const int col = kSplit ? cb * L * C + sub * 4 : (cb * L + sub) * C;
    const bool col_ok = col < f.dim;
    // split rows: piece 1 sits 4L elements after piece 0 (dims are multiples of 8 here)
    const int pieces = kSplit ? (col + 4 * L < f.dim ? 2 : 1) : 0;
    // Two pass groups in flight: the rows of group k+1 are requested before
    // group k is stored, so no row load waits behind a store.
    int64_t nid[kUnroll];  // ids of the next group to load
    auto fetch_ids = [&](int base) {
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const int i = base + u * G + slot;
        nid[u] = i < count ? ids[i] : 0;
      }
    };
    auto load_rows = [&](int base, float (&v)[kUnroll][C]) {
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const int i = base + u * G + slot;
        const bool ok = i < count && (uint64_t)nid[u] < (uint64_t)f.num_rows && col_ok;
        if constexpr (kSplit)
          RowIO<float, C>::load_pieces(ok ? W + nid[u] * f.dim + col : zero_row<float>(), 4 * L, ok ? pieces : 0, v[u]);
        else
          RowIO<TW, C>::load(ok ? W + nid[u] * f.dim + col : zero_row<TW>(), v[u]);
      }
    };
    auto store_rows = [&](int base, const float (&v)[kUnroll][C]) {
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const int i = base + u * G + slot;
        if (i < count && col_ok) {
          if constexpr (kSplit)
            RowIO<float, C>::template store_pieces<kOutPolicy>(out + (first + i) * f.out_stride + col, 4 * L, pieces, v[u]);
          else
            RowIO<TO, C>::template store<kOutPolicy>(out + (first + i) * f.out_stride + col, v[u]);
        }
      }
    };
    float va[kUnroll][C], vb[kUnroll][C];
    fetch_ids(0);
    load_rows(0, va);
    fetch_ids(step);
    for (int base = 0; base < count; base += 2 * step) {
      const bool more = base + step < count;
      if (more) {
        load_rows(base + step, vb);
        fetch_ids(base + 2 * step);
      }
      store_rows(base, va);
      if (!more) break;
      if (base + 2 * step < count) {
        load_rows(base + 2 * step, va);
        fetch_ids(base + 3 * step);
      }
      store_rows(base + step, vb);
    }
  }
  // Sort keys and payloads (and the invalid-id count), one id per lane, the
  // loads of a batch issued before its stores.
  constexpr int kBatch = 4;
  int bad = 0;
  for (int i0 = lane; i0 < count; i0 += kWave * kBatch) {
    int64_t id[kBatch];
#pragma unroll
    for (int q = 0; q < kBatch; ++q) id[q] = i0 + q * kWave < count ? ids[i0 + q * kWave] : 0;
#pragma unroll
    for (int q = 0; q < kBatch; ++q) {
      const int i = i0 + q * kWave;
      if (i >= count) break;
      const bool in_range = (uint64_t)id[q] < (uint64_t)f.num_rows;
      bad += !in_range;
      if (a.keys != nullptr) {
        const int64_t e = f.ids_begin + first + i;
        st_policy<kOutPolicy>(a.keys + e,
                              (in_range && id[q] != f.padding_idx) ? (uint32_t)(f.row_base + id[q]) : a.sentinel);
        st_policy<kOutPolicy>(a.payload + e, (uint32_t)(f.payload_base + first + i));
      }
    }
  }
  if (bad && a.error_count) atomicAdd(a.error_count, bad);
}

// -------------------------------------------------------------- pooled --

// Stage the chunk's bag bounds [0, nb] in LDS, clamped into the feature's own
// id range, so lengths that do not add up to the ids passed can only give
// wrong sums (and an error count), never an out-of-bounds read.  Decreasing
// offsets (negative lengths) are made non-decreasing.
__device__ __forceinline__ int stage_offsets(const Feat& f, int64_t first_bag, int nb, int64_t* s_off,
                                             const FwdArgs& a) {
  const int lane = lane_id();
  const int64_t lo = f.ids_begin, hi = f.ids_begin + f.num_ids;
  int clamped = 0;
  for (int i = lane; i <= nb; i += kWave) {
    const int64_t o = a.offsets[f.bag_base + first_bag + i];
    const int64_t oc = o < lo ? lo : (o > hi ? hi : o);
    clamped += oc != o;
    s_off[i] = oc;
  }
  wave_sync();
  int dec = 0;
  for (int i = lane + 1; i <= nb; i += kWave) dec += s_off[i] < s_off[i - 1];
  if (__ballot(dec != 0) != 0) {
    // Error path: a running maximum makes every bag's bounds ordered.
    if (lane == 0) {
      int64_t m = s_off[0];
      for (int i = 1; i <= nb; ++i) {
        if (s_off[i] < m) s_off[i] = m;
        m = s_off[i];
      }
    }
    wave_sync();
  }
  return clamped + dec;
}

// Last bag b in [0, nb) with off[b] <= e (the bag holding entry e, skipping
// empty bags), by binary search over the staged bounds.
template <typename T>
__device__ __forceinline__ int bag_of(const T* off, int nb, T e) {
  int lo = 0, hi = nb - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (off[mid] <= e) lo = mid;
    else hi = mid - 1;
  }
  return lo;
}

// Per-wave LDS of a pooled chunk.  Bag bounds are relative to the chunk's
// first id.  row[i] is the table row of the chunk's id i (kNoRow: the id
// pools with weight 0) for the first kIdStage ids, so ids are read from HBM
// once, in one coalesced sweep, and the walk's only global loads are the
// table rows; ids past the stage (a chunk of very long bags) are read where
// they are used.
constexpr int kIdStage = 480;
constexpr int64_t kMaxChunkIds = 1ll << 30;
constexpr uint32_t kNoRow = 0xffffffffu;
struct PoolStage {
  int32_t off[kMaxBagsPerChunk + 1];
  float cnt[kMaxBagsPerChunk];
  uint32_t row[kIdStage];
};

// Wave-uniform extent of a staged chunk.
struct PoolChunk {
  int64_t e0;  // first id of the chunk in the packed id array
  int len;     // ids in the chunk
  int lim;     // ids whose rows are staged
};

// Stage the chunk's bag bounds, clamped into the feature's own id range, so
// lengths that do not add up to the ids passed can only give wrong sums (and
// an error count), never an out-of-bounds read; decreasing offsets (negative
// lengths) are made non-decreasing.  Then stage the rows of its ids, counting
// ids outside [0, num_rows) into bad.
__device__ __forceinline__ PoolChunk stage_pooled(const Feat& f, int64_t first_bag, int nb, PoolStage& st,
                                                  const FwdArgs& a, int& bad) {
  const int lane = lane_id();
  const int64_t lo = f.ids_begin, hi = f.ids_begin + f.num_ids;
  const int64_t* offs = a.offsets + f.bag_base + first_bag;
  const int64_t o0 = offs[0];
  PoolChunk pc;
  pc.e0 = o0 < lo ? lo : (o0 > hi ? hi : o0);
  int err = 0;
  for (int i = lane; i <= nb; i += kWave) {
    const int64_t o = offs[i];
    const int64_t oc = o < lo ? lo : (o > hi ? hi : o);
    err += oc != o;
    int64_t r = oc - pc.e0;
    // 2^30 ids in one chunk: cut short and counted (keeps the walk's int
    // arithmetic on positions far from overflow)
    if (r > kMaxChunkIds) {
      r = kMaxChunkIds;
      ++err;
    }
    st.off[i] = (int32_t)(r < -kMaxChunkIds ? -kMaxChunkIds : r);
  }
  wave_sync();
  int dec = 0;
  for (int i = lane + 1; i <= nb; i += kWave) dec += st.off[i] < st.off[i - 1];
  if (__ballot(dec != 0) != 0) {
    // Error path: a running maximum makes every bag's bounds ordered.
    if (lane == 0) {
      int32_t m = st.off[0];
      for (int i = 1; i <= nb; ++i) {
        if (st.off[i] < m) st.off[i] = m;
        m = st.off[i];
      }
    }
    wave_sync();
  }
  err += dec;
  pc.len = uni32(st.off[nb]);
  // Rows are staged as 32-bit values; a table of 2^32 - 1 rows or more
  // reads every id where it is used.
  pc.lim = f.num_rows < (int64_t)kNoRow ? (pc.len < kIdStage ? pc.len : kIdStage) : 0;
  const bool exclude = (f.flags & MDL_FLAG_EXCLUDE_NULL) != 0;
  const bool by_pos = (f.flags & MDL_FLAG_ROWS_BY_POSITION) != 0;
  constexpr int kBatch = 4;  // ids per lane whose loads are issued together
  for (int i0 = lane; i0 < pc.lim; i0 += kWave * kBatch) {
    int64_t id[kBatch];
#pragma unroll
    for (int q = 0; q < kBatch; ++q) id[q] = i0 + q * kWave < pc.lim ? a.ids[pc.e0 + i0 + q * kWave] : 0;
#pragma unroll
    for (int q = 0; q < kBatch; ++q) {
      const int i = i0 + q * kWave;
      if (i < pc.lim) {
        // Rows by position: row e - ids_begin of `weight` is the id slot's
        // row (already-embedded input); the ids only decide the null weights.
        const int64_t row = by_pos ? pc.e0 + i - f.ids_begin : id[q];
        const bool in_range = (uint64_t)row < (uint64_t)f.num_rows;
        err += !in_range;
        st.row[i] = in_range && !(exclude && id[q] == 0) ? (uint32_t)row : kNoRow;
      }
    }
  }
  wave_sync();
  bad += err;
  return pc;
}

// Pooled rows of a chunk are staged in LDS (fp32) while the ids are walked and
// written out after the walk: a store inside the walk would make the next
// row loads wait for it (one in-order counter for loads and stores).
constexpr int kOutStage = 1024;  // staged floats per wave

template <int C>
__device__ __forceinline__ void lds_put(float* p, const float (&v)[C]) {
  if constexpr (C % 4 == 0) {
#pragma unroll
    for (int q = 0; q < C / 4; ++q)
      reinterpret_cast<float4*>(p)[q] = make_float4(v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]);
  } else {
#pragma unroll
    for (int k = 0; k < C; ++k) p[k] = v[k];
  }
}

template <int C>
__device__ __forceinline__ void lds_get(const float* p, float (&v)[C]) {
  if constexpr (C % 4 == 0) {
#pragma unroll
    for (int q = 0; q < C / 4; ++q) {
      const float4 x = reinterpret_cast<const float4*>(p)[q];
      v[4 * q] = x.x; v[4 * q + 1] = x.y; v[4 * q + 2] = x.z; v[4 * q + 3] = x.w;
    }
  } else {
#pragma unroll
    for (int k = 0; k < C; ++k) v[k] = p[k];
  }
}

// Split fp32 rows (see MDL_SPLIT_ROWS): the lane's two 16-byte pieces sit
// at col and col + stride.
template <int C>
__device__ __forceinline__ void lds_put_pieces(float* p, int stride, int pieces, const float (&v)[C]) {
#pragma unroll
  for (int q = 0; q < C / 4; ++q)
    if (q < pieces)
      *reinterpret_cast<float4*>(p + q * stride) = make_float4(v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]);
}

template <int C>
__device__ __forceinline__ void lds_get_pieces(const float* p, int stride, int pieces, float (&v)[C]) {
#pragma unroll
  for (int q = 0; q < C / 4; ++q) {
    const float4 x = q < pieces ? *reinterpret_cast<const float4*>(p + q * stride) : make_float4(0.f, 0.f, 0.f, 0.f);
    v[4 * q] = x.x; v[4 * q + 1] = x.y; v[4 * q + 2] = x.z; v[4 * q + 3] = x.w;
  }
}

template <typename TW, typename TO, int C>
__device__ __forceinline__ void pooled_chunk(const Feat& f, int64_t first_bag, int nb, const PoolStage& st,
                                             const PoolChunk& pc, float* s_out, const FwdArgs& a) {
  // Ids per slot per iteration: 24 row elements per lane in flight (the
  // walk's registers allow it at five waves per SIMD; 16 measured 3% slower).
  constexpr int U = C == 1 ? 4 : (24 / C > 1 ? 24 / C : 1);
  const int lane = lane_id();
  const int len = pc.len;
  const int L = lanes_for(f.dim, C);
  const int G = kWave / L;
  const int slot = lane / L, sub = lane % L;
  const int ncb = (f.dim + L * C - 1) / (L * C);
  const bool exclude = (f.flags & MDL_FLAG_EXCLUDE_NULL) != 0;
  const bool by_pos = (f.flags & MDL_FLAG_ROWS_BY_POSITION) != 0;
  const bool mean = f.pooling == MDL_POOL_MEAN;
  const bool staged = (int64_t)nb * f.dim <= kOutStage;
  const TW* W = static_cast<const TW*>(f.weight);
  TO* out = static_cast<TO*>(f.out);
  constexpr bool kSplit = MDL_SPLIT_ROWS && std::is_same_v<TW, float> && std::is_same_v<TO, float> && C == 8;
  // First column of the lane's elements in column block cb, and (split rows)
  // how many of its two pieces lie inside the row (dims are multiples of 8).
  auto col_of = [&](int cb) { return kSplit ? cb * L * C + sub * 4 : (cb * L + sub) * C; };
  auto pieces_of = [&](int col) { return col + 4 * L < f.dim ? 2 : 1; };
  // This slot's slice [s0, s1) of the chunk's ids.
  const int K = (len + G - 1) / G;
  const int s0 = slot * K;
  const int s1 = s0 + K < len ? s0 + K : len;
  const bool any = s0 < s1;
  const int b0 = any ? bag_of(st.off, nb, s0) : 0;
  const bool cont = any && st.off[b0] < s0;  // the slice starts inside a bag

  // Row of the chunk's id i, or -1 for weight 0.
  auto row_at = [&](int i) -> int64_t {
    if (i < pc.lim) {
      const uint32_t r = st.row[i];
      return r == kNoRow ? -1 : (int64_t)r;
    }
    const int64_t e = pc.e0 + i;
    const int64_t id = a.ids[e];
    const int64_t row = by_pos ? e - f.ids_begin : id;
    return (uint64_t)row < (uint64_t)f.num_rows && !(exclude && id == 0) ? row : -1;
  };

  // Pooled row of bag b from its sum and weight: staged, or stored at once.
  auto emit_row = [&](int bag, const float (&sum)[C], float wsum, int col, bool col_ok, bool emit_cnt) {
    // sums / max(count, 1), the reference's division (src/model.py:570),
    // once per pooled row
    const float den = mean ? fmaxf(wsum, 1.f) : 1.f;
    float r[C];
#pragma unroll
    for (int k = 0; k < C; ++k) r[k] = sum[k] / den;
    if (staged) {
      if (col_ok) {
        if constexpr (kSplit) lds_put_pieces<C>(s_out + bag * f.dim + col, 4 * L, pieces_of(col), r);
        else lds_put<C>(s_out + bag * f.dim + col, r);
      }
      if (emit_cnt) const_cast<PoolStage&>(st).cnt[bag] = wsum;
    } else {
      if (col_ok) {
        if constexpr (kSplit)
          RowIO<float, C>::template store_pieces<kOutPolicy>(out + (first_bag + bag) * f.out_stride + col, 4 * L,
                                                             pieces_of(col), r);
        else
          RowIO<TO, C>::template store<kOutPolicy>(out + (first_bag + bag) * f.out_stride + col, r);
      }
      if (emit_cnt && a.bag_count != nullptr) st_policy(a.bag_count + f.payload_base + first_bag + bag, wsum);
    }
  };

  for (int cb = 0; cb < ncb; ++cb) {
    const int col = col_of(cb);
    const bool col_ok = col < f.dim;
    const int pcs = pieces_of(col);
    const bool emit = cb == 0 && sub == 0;
    float acc[C], hp[C];
    zero_c(acc);
    zero_c(hp);
    float wsum = 0.f, hw = 0.f;
    int hbag = -1;  // first bag of a slice that starts inside it, when it ends in the slice
    bool ended = false;
    int b = b0;
    int bend = any ? st.off[b0 + 1] : 0;
    int64_t nrow[U];  // rows of the next iteration
#pragma unroll
    for (int u = 0; u < U; ++u) nrow[u] = s0 + u < s1 ? row_at(s0 + u) : -1;
    for (int j = s0; j < s1; j += U) {
      float v[U][C], wt[U];
      int64_t row[U];
#pragma unroll
      for (int u = 0; u < U; ++u) row[u] = nrow[u];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const bool live = row[u] >= 0 && j + u < s1;
        wt[u] = live ? 1.f : 0.f;
        if constexpr (kSplit)
          RowIO<float, C>::load_pieces(live && col_ok ? W + row[u] * f.dim + col : zero_row<float>(), 4 * L,
                                       live && col_ok ? pcs : 0, v[u]);
        else
          RowIO<TW, C>::load(live && col_ok ? W + row[u] * f.dim + col : zero_row<TW>(), v[u]);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) nrow[u] = j + U + u < s1 ? row_at(j + U + u) : -1;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int e = j + u;
        if (e >= s1) continue;
#pragma unroll
        for (int k = 0; k < C; ++k) acc[k] += v[u][k];
        wsum += wt[u];
        if (e + 1 == bend) {
          if (st.off[b] >= s0) {
            emit_row(b, acc, wsum, col, col_ok, emit);
          } else {
#pragma unroll
            for (int k = 0; k < C; ++k) hp[k] = acc[k];
            hw = wsum;
            hbag = b;
          }
          ended = true;
          zero_c(acc);
          wsum = 0.f;
          // next non-empty bag
          ++b;
          while (b < nb - 1 && st.off[b + 1] <= e + 1) ++b;
          bend = st.off[b + 1 <= nb ? b + 1 : nb];
        }
      }
    }
    // Join bags that cross slot bounds: slot s exports the partial of the bag
    // open at its end; a slice inside one bag passes the previous export on.
    float o[C];
#pragma unroll
    for (int k = 0; k < C; ++k) o[k] = acc[k];
    float ow = wsum;
    bool pass = cont && !ended;
    for (int d = 1; d < G; d <<= 1) {
      const int src = slot >= d ? lane - d * L : lane;
      const int opass = shfl_i((int)pass, src);
      const float oww = shfl_f(ow, src);
      float ov[C];
#pragma unroll
      for (int k = 0; k < C; ++k) ov[k] = shfl_f(o[k], src);
      if (slot >= d) {
        if (pass) {
#pragma unroll
          for (int k = 0; k < C; ++k) o[k] += ov[k];
          ow += oww;
        }
        pass = pass && opass;
      }
    }
    const int prev = slot > 0 ? lane - L : lane;
    float in[C];
#pragma unroll
    for (int k = 0; k < C; ++k) in[k] = shfl_f(o[k], prev);
    const float inw = shfl_f(ow, prev);
    if (hbag >= 0) {
      float t[C];
#pragma unroll
      for (int k = 0; k < C; ++k) t[k] = in[k] + hp[k];
      emit_row(hbag, t, inw + hw, col, col_ok, emit);
    }
  }
  if (staged) {
    // Flush the staged rows (empty bags pool to zero) and the bag weights.
    wave_sync();
    for (int bb = slot; bb < nb; bb += G) {
      const bool empty = st.off[bb] == st.off[bb + 1];
      for (int cb = 0; cb < ncb; ++cb) {
        const int col = col_of(cb);
        if (col >= f.dim) continue;
        float r[C];
        if constexpr (kSplit) {
          const int pcs = pieces_of(col);
          if (empty) zero_c(r);
          else lds_get_pieces<C>(s_out + bb * f.dim + col, 4 * L, pcs, r);
          RowIO<float, C>::template store_pieces<kOutPolicy>(out + (first_bag + bb) * f.out_stride + col, 4 * L, pcs, r);
        } else {
          if (empty) zero_c(r);
          else lds_get<C>(s_out + bb * f.dim + col, r);
          RowIO<TO, C>::template store<kOutPolicy>(out + (first_bag + bb) * f.out_stride + col, r);
        }
      }
    }
    if (a.bag_count != nullptr)
      for (int i = lane; i < nb; i += kWave)
        st_policy(a.bag_count + f.payload_base + first_bag + i, st.off[i] == st.off[i + 1] ? 0.f : st.cnt[i]);
    return;
  }
  // Empty bags pool to zero.
  for (int bb = slot; bb < nb; bb += G) {
    if (st.off[bb] == st.off[bb + 1]) {
      float z[C];
      zero_c(z);
      for (int cb = 0; cb < ncb; ++cb) {
        const int col = col_of(cb);
        if (col >= f.dim) continue;
        if constexpr (kSplit)
          RowIO<float, C>::template store_pieces<kOutPolicy>(out + (first_bag + bb) * f.out_stride + col, 4 * L,
                                                             pieces_of(col), z);
        else
          RowIO<TO, C>::template store<kOutPolicy>(out + (first_bag + bb) * f.out_stride + col, z);
      }
      if (sub == 0 && a.bag_count != nullptr) st_policy(a.bag_count + f.payload_base + first_bag + bb, 0.f);
    }
  }
}

// A chunk whose bags hold one id each (single-id bags, as c4's): bag b's
// pooled row is the row staged for its id, or zeros for an id that pools with
// weight 0, and its weight is 1 or 0, so the chunk is a gather of the staged
// rows straight to the output rows -- no walk, no staged output, two groups
// of row loads in flight as in gather_chunk.  The rows are 0 + row, the bits
// the walk gives (its sum starts at +0; a mean divides by max(1, 1) = 1).
template <typename TW, typename TO, int C>
__device__ __forceinline__ void unit_bags_chunk(const Feat& f, int64_t first_bag, int nb, const PoolStage& st,
                                                const FwdArgs& a) {
  constexpr int kUnroll = unroll_for<C>();
  const int lane = lane_id();
  const int L = lanes_for(f.dim, C);
  const int G = kWave / L;
  const int slot = lane / L, sub = lane % L;
  const int ncb = (f.dim + L * C - 1) / (L * C);
  const TW* W = static_cast<const TW*>(f.weight);
  TO* out = static_cast<TO*>(f.out);
  const int step = G * kUnroll;
  constexpr bool kSplit = MDL_SPLIT_ROWS && std::is_same_v<TW, float> && std::is_same_v<TO, float> && C == 8;
  for (int cb = 0; cb < ncb; ++cb) {
    const int col = kSplit ? cb * L * C + sub * 4 : (cb * L + sub) * C;
    const bool col_ok = col < f.dim;
    const int pieces = kSplit ? (col + 4 * L < f.dim ? 2 : 1) : 0;
    auto load_rows = [&](int base, float (&v)[kUnroll][C]) {
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const int i = base + u * G + slot;
        const uint32_t r = i < nb ? st.row[i] : kNoRow;
        const bool ok = r != kNoRow && col_ok;
        if constexpr (kSplit)
          RowIO<float, C>::load_pieces(ok ? W + (int64_t)r * f.dim + col : zero_row<float>(), 4 * L,
                                       ok ? pieces : 0, v[u]);
        else
          RowIO<TW, C>::load(ok ? W + (int64_t)r * f.dim + col : zero_row<TW>(), v[u]);
      }
    };
    auto store_rows = [&](int base, const float (&v)[kUnroll][C]) {
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const int i = base + u * G + slot;
        if (i < nb && col_ok) {
          float r[C];
#pragma unroll
          for (int k = 0; k < C; ++k) r[k] = 0.f + v[u][k];
          if constexpr (kSplit)
            RowIO<float, C>::template store_pieces<kOutPolicy>(out + (first_bag + i) * f.out_stride + col, 4 * L,
                                                               pieces, r);
          else
            RowIO<TO, C>::template store<kOutPolicy>(out + (first_bag + i) * f.out_stride + col, r);
        }
      }
    };
    float va[kUnroll][C], vb[kUnroll][C];
    load_rows(0, va);
    for (int base = 0; base < nb; base += 2 * step) {
      const bool more = base + step < nb;
      if (more) load_rows(base + step, vb);
      store_rows(base, va);
      if (!more) break;
      if (base + 2 * step < nb) load_rows(base + 2 * step, va);
      store_rows(base + step, vb);
    }
  }
  if (a.bag_count != nullptr)
    for (int i = lane; i < nb; i += kWave)
      st_policy(a.bag_count + f.payload_base + first_bag + i, st.row[i] != kNoRow ? 1.f : 0.f);
}

// Sort keys and payloads of a pooled chunk, one id per lane so the stores
// coalesce; an id's bag comes from a binary search of the staged bounds,
// resumed from the lane's previous id.  Returns the invalid ids among those
// not staged (the staged ones were counted when staged).
__device__ __forceinline__ int pooled_keys(const Feat& f, int64_t first_bag, int nb, const PoolStage& st,
                                           const PoolChunk& pc, const FwdArgs& a) {
  constexpr int kBatch = 4;  // ids per lane whose loads are issued before any store
  const int lane = lane_id();
  const bool exclude = (f.flags & MDL_FLAG_EXCLUDE_NULL) != 0;
  const bool by_pos = (f.flags & MDL_FLAG_ROWS_BY_POSITION) != 0;
  int bad = 0;
  int b = 0;
  for (int base = lane; base < pc.len; base += kWave * kBatch) {
    int64_t id[kBatch];
#pragma unroll
    for (int q = 0; q < kBatch; ++q) {
      const int i = base + q * kWave;
      id[q] = i < pc.len && i >= pc.lim ? a.ids[pc.e0 + i] : 0;
    }
#pragma unroll
    for (int q = 0; q < kBatch; ++q) {
      const int i = base + q * kWave;
      if (i >= pc.len) break;
      int hi = nb - 1;  // last bag with off[bag] <= i, searched in [b, nb)
      while (b < hi) {
        const int mid = (b + hi + 1) >> 1;
        if (st.off[mid] <= i) b = mid;
        else hi = mid - 1;
      }
      // Invalid ids and nulls under "exclude" pool with weight 0: their
      // gradient is exactly zero, so they take no part in the backward.
      // Rows by position belong to no table.
      int64_t row;
      bool live;
      if (i < pc.lim) {
        const uint32_t r = st.row[i];
        row = (int64_t)r;
        live = r != kNoRow;
      } else {
        const int64_t e = pc.e0 + i;
        row = by_pos ? e - f.ids_begin : id[q];
        const bool in_range = (uint64_t)row < (uint64_t)f.num_rows;
        bad += !in_range;
        live = in_range && !(exclude && id[q] == 0);
      }
      if (a.keys != nullptr) {
        const int64_t e = pc.e0 + i;
        live = live && !by_pos && row != (int64_t)f.padding_idx;
        st_policy<kOutPolicy>(a.keys + e, live ? (uint32_t)(f.row_base + row) : a.sentinel);
        st_policy<kOutPolicy>(a.payload + e, (uint32_t)(f.payload_base + first_bag + b));
      }
    }
  }
  return bad;
}

template <typename TW, typename TO, bool kVec>
__global__ MDL_OCCUPANCY __launch_bounds__(kFwdWaves * kWave) void forward_kernel(FwdArgs a) {
  __shared__ PoolStage s_st[kFwdWaves];
  __shared__ __align__(16) float s_out[kFwdWaves][kOutStage];
  const int w = threadIdx.x / kWave;
  const int64_t blk = xcd_block(blockIdx.x, gridDim.x);
  const int64_t c = uni64(blk * kFwdWaves + w);
  if (c >= a.num_chunks) return;
  mdl_chunk ch;
  ch.feature = uni32(a.chunks[c].feature);
  ch.count = uni32(a.chunks[c].count);
  ch.first = uni64(a.chunks[c].first);
  Feat f = load_feat(a.feats + ch.feature);
  const int v = feat_variant(f);
  if (v / kWidths != ClassOf<TW, TO, kVec>::value) return;  // another class's launch owns it
  if (a.key_origin != nullptr) {
    // This call's ids start at the origin: positions before it are clamped
    // away, and position i lands in entry i - origin.
    int64_t o = uni64(*a.key_origin);
    o = o < 0 ? 0 : (o > a.num_ids ? a.num_ids : o);
    a.key_lo = o;
    if (a.keys != nullptr) {
      a.keys -= o;
      a.payload -= o;
    }
  }
  bind_range(f, a);
  if (f.pooling == MDL_POOL_NONE) {
    // The chunk may reach past a range that is shorter this call.
    const int64_t left = f.num_ids - ch.first;
    const int count = left < (int64_t)ch.count ? (left > 0 ? (int)left : 0) : ch.count;
    if (count > 0)
      with_width<TW, kVec>(v % kWidths, [&]<int C>() { gather_chunk<TW, TO, C>(f, ch.first, count, a); });
    return;
  }
  if (ch.count > kMaxBagsPerChunk || ch.count <= 0) {
    if (lane_id() == 0 && a.error_count && ch.count != 0) atomicAdd(a.error_count, 1);
    return;
  }
  int bad = 0;
  const PoolChunk pc = stage_pooled(f, ch.first, ch.count, s_st[w], a, bad);
  // Every bag of the chunk one id long (bounds 0, 1, ..., nb after staging,
  // every row staged): a gather instead of the walk.
  bool unit = pc.len == ch.count && pc.lim == pc.len;
  if (unit) {
    bool off = false;
    for (int b = lane_id(); b < ch.count; b += kWave) off |= s_st[w].off[b + 1] - s_st[w].off[b] != 1;
    unit = __ballot(off) == 0;
  }
  with_width<TW, kVec>(v % kWidths, [&]<int C>() {
    if (unit) unit_bags_chunk<TW, TO, C>(f, ch.first, ch.count, s_st[w], a);
    else pooled_chunk<TW, TO, C>(f, ch.first, ch.count, s_st[w], pc, s_out[w], a);
  });
  // After the walk, so that its stores never hold up the walk's loads.
  bad += pooled_keys(f, ch.first, ch.count, s_st[w], pc, a);
  for (int m = 1; m < kWave; m <<= 1) bad += __shfl_xor(bad, m);
  if (lane_id() == 0 && bad && a.error_count) atomicAdd(a.error_count, bad);
}

// ------------------------------------------------------ pool backward --

// Per-position gradient of one chunk of bags: slot e of bag b receives the
// bag's upstream gradient row times w_e / max(count_b, 1) (mean) or w_e (sum).
// The walk over the chunk's positions visits consecutive slots of one bag
// together, so they read the same gradient row, which stays in L2: HBM sees
// about one read of each pooled gradient row and one write of each position
// row.
template <typename TW, typename TO, int C>
__device__ __forceinline__ void unpool_chunk(const Feat& f, int64_t first_bag, int nb, int64_t* s_off,
                                             const FwdArgs& a) {
  constexpr int kUnroll = unroll_for<C>();
  const int lane = lane_id();
  stage_offsets(f, first_bag, nb, s_off, a);
  const int64_t e_begin = s_off[0], e_end = s_off[nb];
  const int L = lanes_for(f.dim, C);
  const int G = kWave / L;
  const int slot = lane / L, sub = lane % L;
  const int ncb = (f.dim + L * C - 1) / (L * C);
  const bool exclude = (f.flags & MDL_FLAG_EXCLUDE_NULL) != 0;
  const bool by_pos = (f.flags & MDL_FLAG_ROWS_BY_POSITION) != 0;
  const bool mean = f.pooling == MDL_POOL_MEAN;
  const TO* grad = static_cast<const TO*>(f.out);
  TW* dst = static_cast<TW*>(const_cast<void*>(f.weight));
  const float* counts = a.bag_count + f.payload_base + first_bag;
  const int64_t step = (int64_t)G * kUnroll;
  for (int cb = 0; cb < ncb; ++cb) {
    const int col = (cb * L + sub) * C;
    const bool col_ok = col < f.dim;
    int bag = 0;
    for (int64_t base = e_begin; base < e_end; base += step) {
      int64_t id[kUnroll];
      int bg[kUnroll];
      bool valid[kUnroll];
      float cnt[kUnroll], v[kUnroll][C];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const int64_t e = base + (int64_t)u * G + slot;
        valid[u] = e < e_end;
        id[u] = valid[u] ? a.ids[e] : 0;
        if (valid[u]) {
          while (s_off[bag + 1] <= e) ++bag;
        }
        bg[u] = bag;
      }
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        cnt[u] = *(mean && valid[u] ? counts + bg[u] : zero_row<float>());
        RowIO<TO, C>::load(valid[u] && col_ok ? grad + (first_bag + bg[u]) * f.out_stride + col : zero_row<TO>(),
                           v[u]);
      }
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const int64_t e = base + (int64_t)u * G + slot;
        const int64_t row = e - f.ids_begin;
        // Positions the forward gave weight 0: nulls under "exclude" and rows
        // outside [0, num_rows).
        const int64_t src = by_pos ? row : id[u];
        const bool dead = (exclude && id[u] == 0) || (uint64_t)src >= (uint64_t)f.num_rows;
        // grad / max(count, 1): the autograd of the reference's division
        const BagDivisor div(mean ? fmaxf(cnt[u], 1.f) : 1.f);
#pragma unroll
        for (int k = 0; k < C; ++k) v[u][k] = dead ? 0.f : div(v[u][k]);
        if (valid[u] && col_ok) RowIO<TW, C>::store(dst + row * f.dim + col, v[u]);
      }
    }
  }
}

template <typename TW, typename TO, bool kVec>
__global__ __launch_bounds__(kFwdWaves * kWave) void pool_backward_kernel(FwdArgs a) {
  __shared__ int64_t s_off[kFwdWaves][kMaxBagsPerChunk + 1];
  const int w = threadIdx.x / kWave;
  const int64_t blk = xcd_block(blockIdx.x, gridDim.x);
  const int64_t c = uni64(blk * kFwdWaves + w);
  if (c >= a.num_chunks) return;
  const int32_t fi = uni32(a.chunks[c].feature);
  const int32_t count = uni32(a.chunks[c].count);
  const int64_t first = uni64(a.chunks[c].first);
  Feat f = load_feat(a.feats + fi);
  const int v = feat_variant(f);
  if (v / kWidths != ClassOf<TW, TO, kVec>::value) return;  // another class's launch owns it
  if (f.pooling == MDL_POOL_NONE || count > kMaxBagsPerChunk || count <= 0) return;
  bind_range(f, a);
  with_width<TW, kVec>(v % kWidths, [&]<int C>() { unpool_chunk<TW, TO, C>(f, first, count, s_off[w], a); });
}

struct LaunchForward {
  const FwdArgs& a;
  int64_t blocks;
  hipStream_t s;
  bool backward;
  template <typename TW, typename TO, bool kVec>
  int operator()() const {
    if (backward) {
      hipLaunchKernelGGL((pool_backward_kernel<TW, TO, kVec>), dim3((unsigned)blocks), dim3(kFwdWaves * kWave), 0, s,
                         a);
      MDL_CHECK_LAUNCH("pool_backward_kernel");
    } else {
      hipLaunchKernelGGL((forward_kernel<TW, TO, kVec>), dim3((unsigned)blocks), dim3(kFwdWaves * kWave), 0, s, a);
      MDL_CHECK_LAUNCH("forward_kernel");
    }
    return MDL_OK;
  }
};

// ------------------------------------------------------------ sequences --

struct SeqArgs {
  Feat f;
  const int64_t* ids;
  const int64_t* lengths;
  int64_t batch, in_len, out_len;
  int order;
  void* out;
  uint8_t* mask;
  uint32_t* keys;
  uint32_t* payload;
  const int64_t* key_offsets;  // packed keys: row b's at [key_offsets[b], key_offsets[b + 1])
  uint32_t sentinel;
  int32_t* error_count;
};

// Valid window positions of row b: the length clamped to [0, out_len], and
// none when the input is empty (src/model.py:2998-3011).  A length past the
// input width keeps its positions: each one past the input repeats the last
// input element (the reference clamps the source position to in_len - 1,
// :3014-3016), see seq_src.
__device__ __forceinline__ int64_t seq_len(const SeqArgs& a, int64_t b) {
  if (a.in_len <= 0) return 0;
  int64_t n = a.lengths[b];
  n = n < 0 ? 0 : n;
  return n > a.out_len ? a.out_len : n;
}

// Input position of window entry rel in [0, len) of a row.
__device__ __forceinline__ int64_t seq_src(const SeqArgs& a, int64_t len, int64_t rel) {
  const int64_t k = a.order == MDL_SEQ_OLDEST_TO_NEWEST ? rel : len - 1 - rel;
  return k < a.in_len ? k : a.in_len - 1;
}

// One wave per chunk of kSeqRows output positions [p0, p0 + np) of one row
// b of [batch, out_len]: the chunk's first nz positions are padding (zeros),
// the rest hold the ids of one contiguous (oldest_to_newest) or reversed
// (newest_to_oldest) run of input positions, so the row's length is one
// scalar load and the ids load coalesced.  The gather keeps two pass groups
// of rows in flight, as the unpooled lookup does; padding rows and the mask
// are stored after it, so no row load waits behind those stores.
// Positions per wave: short chunks (about one pass group pair) spread the
// ragged rows evenly over the waves; measured best at 16..48.
#ifndef MDL_SEQ_ROWS
#define MDL_SEQ_ROWS 32
#endif
constexpr int kSeqRows = MDL_SEQ_ROWS;

template <typename TW, typename TO, int C>
__device__ __forceinline__ void seq_chunk(const SeqArgs& a, int64_t b, int64_t p0, int np) {
  constexpr int kUnroll = unroll_for<C>();
  const Feat& f = a.f;
  const int lane = lane_id();
  const int L = lanes_for(f.dim, C);
  const int G = kWave / L;
  const int slot = lane / L, sub = lane % L;
  const int ncb = (f.dim + L * C - 1) / (L * C);
  const TW* W = static_cast<const TW*>(f.weight);
  TO* out = static_cast<TO*>(a.out) + (b * a.out_len + p0) * f.out_stride;
  const int64_t len = uni64(seq_len(a, b));
  const int64_t start = a.out_len - len;
  const int nz = start <= p0 ? 0 : (start - p0 < np ? (int)(start - p0) : np);
  const int count = np - nz;
  const int64_t k0 = p0 + nz - start;  // run position of the chunk's first id
  const int64_t* ids = a.ids + b * a.in_len;
  const int step = G * kUnroll;
  int bad = 0;
  constexpr bool kSplit = MDL_SPLIT_ROWS && std::is_same_v<TW, float> && std::is_same_v<TO, float> && C == 8;
  for (int cb = 0; cb < ncb; ++cb) {
    const int col = kSplit ? cb * L * C + sub * 4 : (cb * L + sub) * C;
    const bool col_ok = col < f.dim;
    const int pieces = col + 4 * L < f.dim ? 2 : 1;  // split rows only
    const bool first = cb == 0 && sub == 0;
    int64_t nid[kUnroll];  // ids of the next group to load
    auto fetch_ids = [&](int base) {
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const int i = base + u * G + slot;
        nid[u] = i < count ? ids[seq_src(a, len, k0 + i)] : 0;
      }
    };
    auto load_rows = [&](int base, float (&v)[kUnroll][C]) {
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const int i = base + u * G + slot;
        const bool in_range = (uint64_t)nid[u] < (uint64_t)f.num_rows;
        if (first && i < count) bad += !in_range;
        const bool ok = i < count && in_range && col_ok;
        if constexpr (kSplit)
          RowIO<float, C>::load_pieces(ok ? W + nid[u] * f.dim + col : zero_row<float>(), 4 * L, ok ? pieces : 0, v[u]);
        else
          RowIO<TW, C>::load(ok ? W + nid[u] * f.dim + col : zero_row<TW>(), v[u]);
      }
    };
    auto store_rows = [&](int base, const float (&v)[kUnroll][C]) {
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const int i = base + u * G + slot;
        if (i < count && col_ok) {
          if constexpr (kSplit)
            RowIO<float, C>::template store_pieces<kOutPolicy>(out + (int64_t)(nz + i) * f.out_stride + col, 4 * L,
                                                               pieces, v[u]);
          else
            RowIO<TO, C>::template store<kOutPolicy>(out + (int64_t)(nz + i) * f.out_stride + col, v[u]);
        }
      }
    };
    float va[kUnroll][C], vb[kUnroll][C];
    fetch_ids(0);
    load_rows(0, va);
    fetch_ids(step);
    for (int base = 0; base < count; base += 2 * step) {
      const bool more = base + step < count;
      if (more) {
        load_rows(base + step, vb);
        fetch_ids(base + 2 * step);
      }
      store_rows(base, va);
      if (!more) break;
      if (base + 2 * step < count) {
        load_rows(base + 2 * step, va);
        fetch_ids(base + 3 * step);
      }
      store_rows(base + step, vb);
    }
    float z[C];
#pragma unroll
    for (int k = 0; k < C; ++k) z[k] = 0.f;
    if (col_ok)
      for (int i = slot; i < nz; i += G) {
        if constexpr (kSplit)
          RowIO<float, C>::template store_pieces<kOutPolicy>(out + (int64_t)i * f.out_stride + col, 4 * L, pieces, z);
        else
          RowIO<TO, C>::template store<kOutPolicy>(out + (int64_t)i * f.out_stride + col, z);
      }
  }
  if (a.mask)
    for (int i = lane; i < np; i += kWave) a.mask[b * a.out_len + p0 + i] = i >= nz ? 1 : 0;
  for (int m = 1; m < kWave; m <<= 1) bad += __shfl_xor(bad, m);
  if (lane == 0 && bad && a.error_count) atomicAdd(a.error_count, bad);
}

template <typename TW, typename TO, bool kVec>
__global__ MDL_OCCUPANCY __launch_bounds__(kFwdWaves * kWave) void sequence_kernel(SeqArgs a, int width) {
  const int w = threadIdx.x / kWave;
  const int64_t blk = xcd_block(blockIdx.x, gridDim.x);
  const int64_t wid = uni64(blk * kFwdWaves + w);
  const int64_t per_row = (a.out_len + kSeqRows - 1) / kSeqRows;
  if (wid >= a.batch * per_row) return;
  const int64_t b = wid / per_row;
  const int64_t p0 = (wid - b * per_row) * kSeqRows;
  const int np = a.out_len - p0 < kSeqRows ? (int)(a.out_len - p0) : kSeqRows;
  with_width<TW, kVec>(width, [&]<int C>() { seq_chunk<TW, TO, C>(a, b, p0, np); });
}

// Sort keys/payloads of the window entries (b, rel), rel in [0, len_b), of a
// sequence feature: entry rel sits at window position p = out_len - len_b +
// rel and reads input position seq_src(rel), so an input element that the
// window repeats gets one entry per position.  One block per kSeqKeys entries
// of one row, so the row's length is one load.  Dense: entry rel of row b at
// b * out_len + rel.  Packed (key_offsets): the row's first cap =
// key_offsets[b + 1] - key_offsets[b] entries (at most out_len) at
// key_offsets[b] + rel, so the sort sees no padding; a row longer than its
// cap loses the rest, a shorter one fills it with sentinels.
constexpr int kSeqKeys = 1024;

__global__ __launch_bounds__(256) void sequence_keys_kernel(SeqArgs a) {
  const int64_t per_row = (a.out_len + kSeqKeys - 1) / kSeqKeys;
  const int64_t b = (int64_t)blockIdx.x / per_row;
  const int64_t kb = ((int64_t)blockIdx.x - b * per_row) * kSeqKeys;
  const int64_t len = seq_len(a, b);
  const int64_t start = a.out_len - len;
  const bool packed = a.key_offsets != nullptr;
  int64_t base = b * a.out_len, cap = a.out_len;
  if (packed) {
    base = a.key_offsets[b];
    cap = a.key_offsets[b + 1] - base;
    cap = cap < 0 ? 0 : (cap > a.out_len ? a.out_len : cap);
  }
  for (int j = threadIdx.x; j < kSeqKeys; j += 256) {
    const int64_t rel = kb + j;
    if (rel >= cap) break;
    const bool in_window = rel < len;
    const int64_t id = in_window ? a.ids[b * a.in_len + seq_src(a, len, rel)] : 0;
    const bool valid = in_window && (uint64_t)id < (uint64_t)a.f.num_rows && id != a.f.padding_idx;
    a.keys[base + rel] = valid ? (uint32_t)(a.f.row_base + id) : a.sentinel;
    a.payload[base + rel] = valid ? (uint32_t)(a.f.payload_base + b * a.out_len + start + rel) : 0u;
  }
}

struct LaunchSequence {
  const SeqArgs& a;
  int64_t blocks;
  int width;
  hipStream_t s;
  template <typename TW, typename TO, bool kVec>
  int operator()() const {
    hipLaunchKernelGGL((sequence_kernel<TW, TO, kVec>), dim3((unsigned)blocks), dim3(kFwdWaves * kWave), 0, s, a,
                       width);
    MDL_CHECK_LAUNCH("sequence_kernel");
    return MDL_OK;
  }
};

}  // namespace mdl

using namespace mdl;

extern "C" {

uint32_t mdl_feature_classes(const mdl_feature* feats, int32_t num_features) {
  uint32_t m = 0;
  for (int32_t i = 0; i < num_features; ++i) {
    const mdl_feature& f = feats[i];
    m |= 1u << variant_of(f.wdtype, f.odtype, feature_vec(f.weight, f.out, f.dim, f.out_stride, f.wdtype, f.odtype),
                          f.dim);
  }
  return m;
}

int64_t mdl_plan_chunks(const mdl_feature* feats, int32_t num_features, int32_t target_ids,
                        mdl_chunk* chunks, int64_t capacity) {
  if (num_features < 0 || target_ids <= 0) return fail(MDL_ERR_INVALID, "mdl_plan_chunks: bad arguments");
  int64_t n = 0;
  for (int32_t fi = 0; fi < num_features; ++fi) {
    const mdl_feature& f = feats[fi];
    // Rows a wave holds at once (same lane layout as the kernel): chunks hold
    // about kFwdPassesPerChunk of them per slot, so no slot walks a long serial
    // chain of dependent loads, whatever the row width.
    const bool vec = feature_vec(f.weight, f.out, f.dim, f.out_stride, f.wdtype, f.odtype);
    const int c = variant_elems(variant_of(f.wdtype, f.odtype, vec, f.dim));
    const int lanes = lanes_for(f.dim > 0 ? f.dim : 1, c);
    const int64_t per_pass = kWave / lanes;
    int64_t target = (int64_t)kFwdPassesPerChunk * per_pass;
    if (target > target_ids) target = target_ids;
    if (f.pooling == MDL_POOL_NONE) {
      for (int64_t s = 0; s < f.num_ids; s += target) {
        if (chunks && n < capacity) {
          chunks[n].feature = fi;
          chunks[n].first = s;
          chunks[n].count = (int32_t)(f.num_ids - s < target ? f.num_ids - s : target);
        }
        ++n;
      }
    } else {
      const double avg = f.num_bags > 0 ? (double)f.num_ids / (double)f.num_bags : 1.0;
      int64_t nb = 1;
      while (nb * 2 <= kMaxBagsPerChunk && (double)(nb * 2) * (avg > 1.0 ? avg : 1.0) <= (double)target) nb *= 2;
      for (int64_t s = 0; s < f.num_bags; s += nb) {
        if (chunks && n < capacity) {
          chunks[n].feature = fi;
          chunks[n].first = s;
          chunks[n].count = (int32_t)(f.num_bags - s < nb ? f.num_bags - s : nb);
        }
        ++n;
      }
    }
  }
  return n;
}

int mdl_forward(const mdl_feature* feats, int32_t num_features, const mdl_chunk* chunks,
                int64_t num_chunks, const int64_t* ids, int64_t num_ids, const int64_t* offsets,
                uint32_t* sort_keys, uint32_t* sort_payload, const int64_t* key_origin, uint32_t sentinel,
                float* bag_count, int32_t* error_count, uint32_t classes, void* stream) {
  if (num_features < 0 || num_chunks < 0 || num_ids < 0)
    return fail(MDL_ERR_INVALID, "mdl_forward: negative count");
  if (num_chunks == 0) return MDL_OK;
  if (!feats || !chunks || !ids) return fail(MDL_ERR_INVALID, "mdl_forward: null pointer");
  if ((sort_keys == nullptr) != (sort_payload == nullptr))
    return fail(MDL_ERR_INVALID, "mdl_forward: sort_keys and sort_payload go together");
  FwdArgs a;
  a.feats = feats;
  a.chunks = chunks;
  a.num_chunks = num_chunks;
  a.ids = ids;
  a.num_ids = num_ids;
  a.offsets = offsets;
  a.keys = sort_keys;
  a.payload = sort_payload;
  a.key_origin = key_origin;
  a.key_lo = 0;
  a.bag_count = bag_count;
  a.error_count = error_count;
  a.sentinel = sentinel;
  const int64_t blocks = (num_chunks + kFwdWaves - 1) / kFwdWaves;
  if (blocks > 0x7fffffff) return fail(MDL_ERR_UNSUPPORTED, "mdl_forward: too many chunks");
  return for_each_class(classes, LaunchForward{a, blocks, as_stream(stream), false});
}

int mdl_pool_backward(const mdl_feature* feats, int32_t num_features, const mdl_chunk* chunks,
                      int64_t num_chunks, const int64_t* ids, int64_t num_ids, const int64_t* offsets,
                      const float* bag_count, uint32_t classes, void* stream) {
  if (num_features < 0 || num_chunks < 0 || num_ids < 0)
    return fail(MDL_ERR_INVALID, "mdl_pool_backward: negative count");
  if (num_chunks == 0) return MDL_OK;
  if (!feats || !chunks || !ids || !offsets || !bag_count)
    return fail(MDL_ERR_INVALID, "mdl_pool_backward: null pointer");
  FwdArgs a;
  a.feats = feats;
  a.chunks = chunks;
  a.num_chunks = num_chunks;
  a.ids = ids;
  a.num_ids = num_ids;
  a.offsets = offsets;
  a.keys = nullptr;
  a.payload = nullptr;
  a.key_origin = nullptr;
  a.key_lo = 0;
  a.bag_count = const_cast<float*>(bag_count);
  a.error_count = nullptr;
  a.sentinel = 0;
  const int64_t blocks = (num_chunks + kFwdWaves - 1) / kFwdWaves;
  if (blocks > 0x7fffffff) return fail(MDL_ERR_UNSUPPORTED, "mdl_pool_backward: too many chunks");
  return for_each_class(classes, LaunchForward{a, blocks, as_stream(stream), true});
}

int mdl_sequence_forward(const mdl_feature* feature, const int64_t* ids, const int64_t* lengths,
                         int64_t batch, int64_t in_len, int64_t out_len, int32_t order, void* out,
                         uint8_t* mask, uint32_t* sort_keys, uint32_t* sort_payload,
                         const int64_t* key_offsets, uint32_t sentinel, int32_t* error_count,
                         void* stream) {
  if (!feature || batch < 0 || in_len < 0 || out_len < 0)
    return fail(MDL_ERR_INVALID, "mdl_sequence_forward: bad arguments");
  if (order != MDL_SEQ_OLDEST_TO_NEWEST && order != MDL_SEQ_NEWEST_TO_OLDEST)
    return fail(MDL_ERR_INVALID, "mdl_sequence_forward: bad order");
  if ((sort_keys == nullptr) != (sort_payload == nullptr))
    return fail(MDL_ERR_INVALID, "mdl_sequence_forward: sort_keys and sort_payload go together");
  SeqArgs a;
  const mdl_feature& d = *feature;
  a.f.weight = (const void*)d.weight;
  a.f.out = out;
  a.f.num_rows = d.num_rows;
  a.f.out_stride = d.dim;
  a.f.row_base = d.row_base;
  a.f.payload_base = d.payload_base;
  a.f.ids_begin = 0;
  a.f.bag_base = 0;
  a.f.dim = d.dim;
  a.f.wdtype = d.wdtype;
  a.f.odtype = d.odtype;
  a.f.pooling = MDL_POOL_NONE;
  a.f.flags = d.flags;
  a.f.padding_idx = d.padding_idx;
  if (d.dim <= 0) return fail(MDL_ERR_INVALID, "mdl_sequence_forward: dim must be positive");
  if (d.wdtype == MDL_F32 && d.odtype != MDL_F32)
    return fail(MDL_ERR_UNSUPPORTED, "mdl_sequence_forward: fp32 weights need fp32 output");
  a.ids = ids;
  a.lengths = lengths;
  a.batch = batch;
  a.in_len = in_len;
  a.out_len = out_len;
  a.order = order;
  a.out = out;
  a.mask = mask;
  a.keys = sort_keys;
  a.payload = sort_payload;
  a.key_offsets = key_offsets;
  a.sentinel = sentinel;
  a.error_count = error_count;
  hipStream_t s = as_stream(stream);
  if (batch > 0 && out_len > 0) {
    const int64_t waves = batch * ((out_len + kSeqRows - 1) / kSeqRows);
    const int64_t blocks = (waves + kFwdWaves - 1) / kFwdWaves;
    if (blocks > 0x7fffffff) return fail(MDL_ERR_UNSUPPORTED, "mdl_sequence_forward: too many rows");
    const bool vec = feature_vec(d.weight, (uint64_t)out, d.dim, d.dim, d.wdtype, d.odtype);
    const int v = variant_of(d.wdtype, d.odtype, vec, d.dim);
    const int rc = for_each_class(1u << v, LaunchSequence{a, blocks, v % kWidths, s});
    if (rc != MDL_OK) return rc;
  }
  if (sort_keys != nullptr && batch > 0 && out_len > 0) {
    const int64_t blocks = batch * ((out_len + kSeqKeys - 1) / kSeqKeys);
    if (blocks > 0x7fffffff) return fail(MDL_ERR_UNSUPPORTED, "mdl_sequence_forward: too many positions");
    hipLaunchKernelGGL(sequence_keys_kernel, dim3((unsigned)blocks), dim3(256), 0, s, a);
    MDL_CHECK_LAUNCH("sequence_keys_kernel");
  }
  return MDL_OK;
}

}  // extern "C"
