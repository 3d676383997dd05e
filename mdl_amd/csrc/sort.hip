// Stable LSD radix sort of (uint32 key, uint32 payload) pairs and the
// torch.unique-style dedup built on it.
//
// Each 8-bit pass is three launches:
//   upsweep   - per-tile digit histogram  -> counts[digit][tile]
//   scan      - one block per digit scans its row of counts (tile order)
//   downsweep - ranks the tile's keys stably, stages them in LDS in digit
//               order and writes each digit's run to its global slot.
// Ranking inside a wavefront uses ballots: the lanes that share a digit are
// found by intersecting one ballot per digit bit, and a key's rank is the
// popcount of its peers on lower lanes plus the wave's running count of that
// digit.  Keys are visited in index order (item-major, then lane), so equal
// keys keep their input order; that stability is what makes the later
// segment reduction of duplicate rows deterministic.
#include "common.cuh"

namespace mdl {

constexpr int kSortThreads = 256;
constexpr int kSortWaves = kSortThreads / kWave;
// Keys per thread: 16 (4096-entry tiles) when that still gives a few blocks
// per CU, else 8 or 4, so a small sort (c0, c4: ~0.5 M keys) still spreads
// over every CU.  (At c1, 8 M keys, 16 per thread sorts in 0.180 ms, 8 in
// 0.195, 4 in 0.248: the larger tiles' longer digit runs win once the chip
// is full; 32, 8192-key tiles whose 64 KB stage leaves two blocks per CU,
// in 0.214, its downsweep 37.7 us per pass against 30.3.)
#ifndef MDL_SORT_MIN_TILES
#define MDL_SORT_MIN_TILES 512
#endif
constexpr int kMinTiles = MDL_SORT_MIN_TILES;
#ifndef MDL_SORT_MAX_ITEMS
#define MDL_SORT_MAX_ITEMS 16
#endif
static inline int sort_items(int64_t n) {
  for (int items = MDL_SORT_MAX_ITEMS; items > 4; items >>= 1)
    if ((n + kSortThreads * items - 1) / (kSortThreads * items) >= kMinTiles) return items;
  return 4;
}
constexpr int kDigitBits = 8;
constexpr int kRadix = 1 << kDigitBits;

// Entries a pass sorts: n_cap, or the count in device memory (clamped to
// [0, n_cap]) when the caller passes one.  Every launch of a sort is sized
// for n_cap; the blocks past the live tile count return at once, so a sort
// whose size is only known on the device needs no host round trip.
__device__ __forceinline__ int64_t live_count(int64_t n_cap, const int64_t* n_dev) {
  if (n_dev == nullptr) return n_cap;
  const int64_t n = *n_dev;
  return n < 0 ? 0 : (n > n_cap ? n_cap : n);
}

template <int kSortItems>
__device__ __forceinline__ int live_tiles(int64_t n) {
  constexpr int64_t kTile = (int64_t)kSortThreads * kSortItems;
  return (int)((n + kTile - 1) / kTile);
}

// Exclusive scan of one value per thread over a block of kSortThreads:
// shuffles inside each wave, one barrier for the wave totals.  smem holds at
// least kSortWaves words.
__device__ __forceinline__ uint32_t block_exclusive_scan_u32(uint32_t v, uint32_t* smem) {
  const int tid = threadIdx.x, lane = lane_id(), w = tid / kWave;
  uint32_t x = v;
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    const uint32_t o = shfl_u(x, lane >= d ? lane - d : lane);
    if (lane >= d) x += o;
  }
  if (lane == kWave - 1) smem[w] = x;
  __syncthreads();
  uint32_t before = 0;
#pragma unroll
  for (int q = 0; q < kSortWaves; ++q) before += q < w ? smem[q] : 0u;
  __syncthreads();
  return before + x - v;
}

template <int kSortItems>
__global__ __launch_bounds__(kSortThreads) void radix_upsweep(const uint32_t* __restrict__ keys, int64_t n_cap,
                                                              const int64_t* __restrict__ n_dev, int shift,
                                                              uint32_t mask, uint32_t* __restrict__ counts) {
  __shared__ uint32_t hist[kSortWaves][kRadix];
  const int64_t n = live_count(n_cap, n_dev);
  const int ntiles = live_tiles<kSortItems>(n);
  if ((int)blockIdx.x >= ntiles) return;
  const int tid = threadIdx.x, w = tid / kWave;
  for (int i = tid; i < kSortWaves * kRadix; i += kSortThreads) (&hist[0][0])[i] = 0u;
  __syncthreads();
  // Consecutive tiles run on one XCD, so the partial lines each tile writes
  // (its counts column here, its digit runs in the downsweep) meet their
  // neighbours in that XCD's L2 before they are written back.
  const int tile = (int)xcd_block(blockIdx.x, ntiles);
  constexpr int kSortTile = kSortThreads * kSortItems;
  const int64_t base = (int64_t)tile * kSortTile;
  uint32_t k[kSortItems];
#pragma unroll
  for (int i = 0; i < kSortItems; ++i) {
    const int64_t idx = base + (int64_t)i * kSortThreads + tid;
    k[i] = keys[idx < n ? idx : n - 1];  // past n: a valid address, not counted
  }
  // A run of neighbouring lanes with one digit adds its length once, from
  // its first lane.  Hot ids (Zipf) sit next to each other once the keys are
  // ordered by their low digits, and the high digits change rarely between
  // neighbours; one LDS atomic per lane would serialise those lanes on one
  // address.
  const int lane = lane_id();
#pragma unroll
  for (int i = 0; i < kSortItems; ++i) {
    const int64_t idx = base + (int64_t)i * kSortThreads + tid;
    const bool valid = idx < n;
    const uint32_t d = (k[i] >> shift) & mask;
    const uint32_t dprev = shfl_u(d, lane > 0 ? lane - 1 : 0);
    const bool head = valid && (lane == 0 || d != dprev);
    const uint64_t heads = __ballot(head);
    const uint32_t nvalid = (uint32_t)__popcll(__ballot(valid));
    if (head) {
      const uint64_t after = heads & ~((2ull << lane) - 1ull);
      const uint32_t end = after ? (uint32_t)__builtin_ctzll(after) : nvalid;
      atomicAdd(&hist[w][d], end - (uint32_t)lane);
    }
  }
  __syncthreads();
  uint32_t s = 0;
#pragma unroll
  for (int q = 0; q < kSortWaves; ++q) s += hist[q][tid];
  counts[(int64_t)tid * ntiles + tile] = s;
}

// Exclusive scan of counts[d][0..ntiles) for digit d = blockIdx.x.
template <int kSortItems>
__global__ __launch_bounds__(kSortThreads) void radix_scan(uint32_t* __restrict__ counts, int64_t n_cap,
                                                           const int64_t* __restrict__ n_dev,
                                                           uint32_t* __restrict__ digit_total) {
  __shared__ uint32_t smem[kSortThreads];
  const int ntiles = live_tiles<kSortItems>(live_count(n_cap, n_dev));
  uint32_t* row = counts + (int64_t)blockIdx.x * ntiles;
  uint32_t carry = 0;
  constexpr int kPer = 4;
  for (int base = 0; base < ntiles; base += kSortThreads * kPer) {
    uint32_t v[kPer];
    uint32_t s = 0;
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const int i = base + threadIdx.x * kPer + k;
      v[k] = i < ntiles ? row[i] : 0u;
      s += v[k];
    }
    const uint32_t ex = block_exclusive_scan_u32(s, smem);
    __shared__ uint32_t s_total;
    if (threadIdx.x == kSortThreads - 1) s_total = ex + s;
    __syncthreads();
    uint32_t run = carry + ex;
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const int i = base + threadIdx.x * kPer + k;
      if (i < ntiles) row[i] = run;
      run += v[k];
    }
    carry += s_total;
    __syncthreads();
  }
  if (threadIdx.x == 0) digit_total[blockIdx.x] = carry;
}

template <int kSortItems>
__global__ __launch_bounds__(kSortThreads) __attribute__((amdgpu_waves_per_eu(4))) void radix_downsweep(
    const uint32_t* __restrict__ keys_in, const uint32_t* __restrict__ vals_in,
    uint32_t* __restrict__ keys_out, uint32_t* __restrict__ vals_out, int64_t n_cap,
    const int64_t* __restrict__ n_dev, int shift, int bits, const uint32_t* __restrict__ counts,
    const uint32_t* __restrict__ digit_total) {
  constexpr int kSortTile = kSortThreads * kSortItems;
  const int64_t n = live_count(n_cap, n_dev);
  const int ntiles = live_tiles<kSortItems>(n);
  if ((int)blockIdx.x >= ntiles) return;
  __shared__ uint32_t s_keys[kSortTile];
  __shared__ uint32_t s_vals[kSortTile];
  __shared__ uint32_t s_wh[kSortWaves][kRadix];
  __shared__ uint32_t s_tile[kRadix];
  __shared__ uint32_t s_gbase[kRadix];
  __shared__ uint32_t s_scan[kSortThreads];

  const int tid = threadIdx.x, w = tid / kWave, lane = tid % kWave;
  const uint32_t mask = (bits >= 32) ? 0xffffffffu : ((1u << bits) - 1u);
  for (int i = tid; i < kSortWaves * kRadix; i += kSortThreads) (&s_wh[0][0])[i] = 0u;
  // This tile's offset inside each digit and the digit totals, requested now
  // and used after the ranking (thread d owns digit d; kSortThreads == kRadix).
  const int tile = (int)xcd_block(blockIdx.x, ntiles);
  const uint32_t my_count_off = counts[(int64_t)tid * ntiles + tile];
  const uint32_t my_total = digit_total[tid];
  __syncthreads();

  const int64_t tile_base = (int64_t)tile * kSortTile;
  const int64_t wave_base = tile_base + (int64_t)w * (kWave * kSortItems);
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  uint32_t k[kSortItems], v[kSortItems], rank[kSortItems];
  // Entries past n (the last tile only) load entry n - 1 instead of
  // branching around the load; the ranking and scatter skip them.
#pragma unroll
  for (int i = 0; i < kSortItems; ++i) {
    const int64_t idx = wave_base + (int64_t)i * kWave + lane;
    const int64_t ic = idx < n ? idx : n - 1;
    k[i] = keys_in[ic];
    v[i] = vals_in[ic];
  }
#pragma unroll
  for (int i = 0; i < kSortItems; ++i) {
    const int64_t idx = wave_base + (int64_t)i * kWave + lane;
    const bool valid = idx < n;
    const uint32_t d = (k[i] >> shift) & mask;
    uint64_t m = __ballot(valid);
    // Always eight ballots, unrolled: a narrower last digit has zero high
    // bits in every lane, whose ballots leave m unchanged.  The lanes that
    // differ from this lane in bit b are ballot ^ t, t all ones when the
    // lane's bit is set; x gathers them with one three-input logic op per
    // half (bitop3 table 0xF6: x | (ballot ^ t)).
    uint32_t t[kDigitBits];
    uint64_t bb[kDigitBits];
#pragma unroll
    for (int b = 0; b < kDigitBits; ++b) {
      t[b] = (uint32_t)((int32_t)(d << (31 - b)) >> 31);
      bb[b] = __ballot(t[b] != 0u);
    }
    uint32_t xlo = 0u, xhi = 0u;
#pragma unroll
    for (int b = 0; b < kDigitBits; ++b) {
      xlo = __builtin_amdgcn_bitop3_b32(xlo, (uint32_t)bb[b], t[b], 0xF6);
      xhi = __builtin_amdgcn_bitop3_b32(xhi, (uint32_t)(bb[b] >> 32), t[b], 0xF6);
    }
    m &= ~(((uint64_t)xhi << 32) | xlo);
    const uint32_t r = (uint32_t)__popcll(m & lt_mask);
    const uint32_t cnt = (uint32_t)__popcll(m);
    const uint32_t old = s_wh[w][d];
    __builtin_amdgcn_wave_barrier();
    if (valid && r == 0) s_wh[w][d] = old + cnt;
    __builtin_amdgcn_wave_barrier();
    rank[i] = old + r;
  }
  __syncthreads();
  {
    const int d = tid;  // kSortThreads == kRadix
    uint32_t run = 0;
#pragma unroll
    for (int q = 0; q < kSortWaves; ++q) {
      const uint32_t c = s_wh[q][d];
      s_wh[q][d] = run;
      run += c;
    }
    const uint32_t tile_prefix = block_exclusive_scan_u32(run, s_scan);
    const uint32_t global_prefix = block_exclusive_scan_u32(my_total, s_scan);
    s_tile[d] = tile_prefix;
    s_gbase[d] = global_prefix + my_count_off - tile_prefix;
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kSortItems; ++i) {
    const int64_t idx = wave_base + (int64_t)i * kWave + lane;
    if (idx < n) {
      const uint32_t d = (k[i] >> shift) & mask;
      const uint32_t pos = s_tile[d] + s_wh[w][d] + rank[i];
      s_keys[pos] = k[i];
      s_vals[pos] = v[i];
    }
  }
  __syncthreads();
  const int64_t rem = n - tile_base;
  const int tile_n = rem < kSortTile ? (int)rem : kSortTile;
  for (int j = tid; j < tile_n; j += kSortThreads) {
    const uint32_t kk = s_keys[j];
    const uint32_t d = (kk >> shift) & mask;
    const uint32_t g = s_gbase[d] + (uint32_t)j;
    keys_out[g] = kk;
    vals_out[g] = s_vals[j];
  }
}

// Passes sort_pairs makes for keys of key_bits bits: the sorted pairs end in
// the alternate buffers when it is odd.
int sort_pass_count(int key_bits) { return key_bits > 0 ? (key_bits + kDigitBits - 1) / kDigitBits : 0; }

// Sized for the smallest tiles (4 keys per thread), so the size never
// decreases with n and a workspace for the largest call serves every smaller
// one.
size_t sort_ws_bytes(int64_t n) {
  const int64_t tile = (int64_t)kSortThreads * 4;
  const int64_t ntiles = (n + tile - 1) / tile;
  return (size_t)(kRadix * (ntiles > 0 ? ntiles : 1) + kRadix) * sizeof(uint32_t) + 256;
}

template <int kSortItems>
static void radix_pass(const uint32_t* ki, const uint32_t* vi, uint32_t* ko, uint32_t* vo, int64_t n,
                       const int64_t* n_dev, int shift, int bits, uint32_t* counts, uint32_t* digit_total,
                       int ntiles, hipStream_t s) {
  const uint32_t mask = (1u << bits) - 1u;
  hipLaunchKernelGGL(radix_upsweep<kSortItems>, dim3(ntiles), dim3(kSortThreads), 0, s, ki, n, n_dev, shift, mask,
                     counts);
  hipLaunchKernelGGL(radix_scan<kSortItems>, dim3(kRadix), dim3(kSortThreads), 0, s, counts, n, n_dev,
                     digit_total);
  hipLaunchKernelGGL(radix_downsweep<kSortItems>, dim3(ntiles), dim3(kSortThreads), 0, s, ki, vi, ko, vo, n,
                     n_dev, shift, bits, counts, digit_total);
}

// n is the capacity (launch sizes, workspace); n_dev, when not null, holds
// the entries actually present (clamped to [0, n]).  The tile size follows
// n, so a count read on the device sorts with the tiles of its capacity.
int sort_pairs(uint32_t* keys, uint32_t* vals, uint32_t* keys_alt, uint32_t* vals_alt, int64_t n,
               const int64_t* n_dev, int key_bits, void* ws, size_t ws_bytes, int* in_alt, hipStream_t s) {
  *in_alt = 0;
  if (n <= 0 || key_bits <= 0) return MDL_OK;
  if (n > 0xffffffffll) return fail(MDL_ERR_UNSUPPORTED, "radix sort: more than 2^32-1 keys");
  if (key_bits > 32) return fail(MDL_ERR_INVALID, "radix sort: key_bits > 32");
  if (ws_bytes < sort_ws_bytes(n)) return fail(MDL_ERR_WORKSPACE, "radix sort: workspace too small");
  const int items = sort_items(n);
  const int ntiles = (int)((n + (int64_t)kSortThreads * items - 1) / ((int64_t)kSortThreads * items));
  uint32_t* counts = static_cast<uint32_t*>(ws);
  uint32_t* digit_total = counts + (size_t)kRadix * ntiles;
  uint32_t* ki = keys;
  uint32_t* vi = vals;
  uint32_t* ko = keys_alt;
  uint32_t* vo = vals_alt;
  int passes = 0;
  for (int shift = 0; shift < key_bits; shift += kDigitBits) {
    const int bits = key_bits - shift < kDigitBits ? key_bits - shift : kDigitBits;
#if MDL_SORT_MAX_ITEMS >= 32
    if (items == 32) radix_pass<32>(ki, vi, ko, vo, n, n_dev, shift, bits, counts, digit_total, ntiles, s);
    else
#endif
    if (items == 16) radix_pass<16>(ki, vi, ko, vo, n, n_dev, shift, bits, counts, digit_total, ntiles, s);
    else if (items == 8) radix_pass<8>(ki, vi, ko, vo, n, n_dev, shift, bits, counts, digit_total, ntiles, s);
    else radix_pass<4>(ki, vi, ko, vo, n, n_dev, shift, bits, counts, digit_total, ntiles, s);
    MDL_CHECK_LAUNCH("radix pass");
    uint32_t* t;
    t = ki; ki = ko; ko = t;
    t = vi; vi = vo; vo = t;
    ++passes;
  }
  *in_alt = passes & 1;  // passes == sort_pass_count(key_bits)
  return MDL_OK;
}

// --------------------------------------------------------------- unique --

__global__ void unique_init(const int64_t* __restrict__ ids, int64_t n, uint32_t* __restrict__ keys,
                            uint32_t* __restrict__ pos) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    keys[i] = (uint32_t)ids[i];
    pos[i] = (uint32_t)i;
  }
}

__global__ void unique_flags(const uint32_t* __restrict__ keys, int64_t n, int64_t* __restrict__ flags) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    flags[i] = (i == 0 || keys[i] != keys[i - 1]) ? 1 : 0;
}

// offs = inclusive positions (n+1 entries, offs[i+1] = heads in [0, i]).
__global__ void unique_scatter(const uint32_t* __restrict__ keys, const uint32_t* __restrict__ pos, int64_t n,
                               const int64_t* __restrict__ offs, int64_t* __restrict__ uniq,
                               int64_t* __restrict__ inverse, int64_t* __restrict__ starts,
                               int64_t* __restrict__ num_unique) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t s = offs[i + 1] - 1;
    if (i == 0 || keys[i] != keys[i - 1]) {
      uniq[s] = keys[i];
      if (starts) starts[s] = i;
    }
    inverse[pos[i]] = s;
    if (i == n - 1) *num_unique = offs[n];
  }
}

__global__ void unique_counts(const uint32_t* __restrict__ keys, int64_t n, const int64_t* __restrict__ offs,
                              int64_t* __restrict__ counts) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    if (i == n - 1 || keys[i + 1] != keys[i]) {
      const int64_t s = offs[i + 1] - 1;
      counts[s] = i + 1 - counts[s];
    }
  }
}

__global__ void write_zero_i64(int64_t* p) { *p = 0; }

static inline unsigned grid_for(int64_t n) {
  int64_t b = (n + 255) / 256;
  if (b < 1) b = 1;
  if (b > 65536) b = 65536;
  return (unsigned)b;
}

}  // namespace mdl

using namespace mdl;

extern "C" {

size_t mdl_sort_workspace_bytes(int64_t n) { return sort_ws_bytes(n); }

int mdl_sort_pairs(uint32_t* keys, uint32_t* payload, uint32_t* keys_alt, uint32_t* payload_alt, int64_t n,
                   int32_t key_bits, void* workspace, size_t workspace_bytes, int32_t* result_in_alt,
                   void* stream) {
  int in_alt = 0;
  int rc = sort_pairs(keys, payload, keys_alt, payload_alt, n, nullptr, key_bits, workspace, workspace_bytes,
                      &in_alt, as_stream(stream));
  if (result_in_alt) *result_in_alt = in_alt;
  return rc;
}

size_t mdl_unique_workspace_bytes(int64_t n) {
  const size_t nn = (size_t)(n > 0 ? n : 1);
  return 4 * nn * sizeof(uint32_t) + nn * sizeof(int64_t) + (nn + 1) * sizeof(int64_t) +
         mdl_offsets_workspace_bytes((int64_t)nn) + sort_ws_bytes((int64_t)nn) + 4 * 256;
}

int mdl_unique(const int64_t* ids, int64_t n, int32_t key_bits, int64_t* unique_out, int64_t* inverse_out,
               int64_t* counts_out, int64_t* num_unique, void* workspace, size_t workspace_bytes,
               void* stream) {
  hipStream_t s = as_stream(stream);
  if (n < 0 || key_bits < 0 || key_bits > 32) return fail(MDL_ERR_INVALID, "mdl_unique: bad arguments");
  if (n == 0) {
    hipLaunchKernelGGL(write_zero_i64, dim3(1), dim3(1), 0, s, num_unique);
    MDL_CHECK_LAUNCH("write_zero_i64");
    return MDL_OK;
  }
  if (workspace_bytes < mdl_unique_workspace_bytes(n)) return fail(MDL_ERR_WORKSPACE, "mdl_unique: workspace too small");
  char* p = static_cast<char*>(workspace);
  auto take = [&](size_t bytes) {
    char* r = p;
    p += (bytes + 255) & ~size_t(255);
    return r;
  };
  uint32_t* k0 = (uint32_t*)take(n * 4);
  uint32_t* v0 = (uint32_t*)take(n * 4);
  uint32_t* k1 = (uint32_t*)take(n * 4);
  uint32_t* v1 = (uint32_t*)take(n * 4);
  int64_t* flags = (int64_t*)take(n * 8);
  int64_t* offs = (int64_t*)take((n + 1) * 8);
  void* scan_ws = take(mdl_offsets_workspace_bytes(n));
  void* sort_ws = take(sort_ws_bytes(n));
  (void)workspace_bytes;
  hipLaunchKernelGGL(unique_init, dim3(grid_for(n)), dim3(256), 0, s, ids, n, k0, v0);
  MDL_CHECK_LAUNCH("unique_init");
  int in_alt = 0;
  int rc = sort_pairs(k0, v0, k1, v1, n, nullptr, key_bits, sort_ws, sort_ws_bytes(n), &in_alt, s);
  if (rc) return rc;
  uint32_t* ks = in_alt ? k1 : k0;
  uint32_t* vs = in_alt ? v1 : v0;
  hipLaunchKernelGGL(unique_flags, dim3(grid_for(n)), dim3(256), 0, s, ks, n, flags);
  MDL_CHECK_LAUNCH("unique_flags");
  rc = mdl_lengths_to_offsets(flags, n, offs, scan_ws, mdl_offsets_workspace_bytes(n), stream);
  if (rc) return rc;
  hipLaunchKernelGGL(unique_scatter, dim3(grid_for(n)), dim3(256), 0, s, ks, vs, n, offs, unique_out,
                     inverse_out, counts_out, num_unique);
  MDL_CHECK_LAUNCH("unique_scatter");
  if (counts_out) {
    hipLaunchKernelGGL(unique_counts, dim3(grid_for(n)), dim3(256), 0, s, ks, n, offs, counts_out);
    MDL_CHECK_LAUNCH("unique_counts");
  }
  return MDL_OK;
}

}  // extern "C"
