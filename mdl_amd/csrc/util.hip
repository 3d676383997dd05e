// Error state, bucketing and the lengths -> offsets scan.
#include "common.cuh"

#include <cstdio>

namespace mdl {

static thread_local std::string g_last_error;

void set_error(const std::string& msg) { g_last_error = msg; }

int fail(int code, const std::string& msg) {
  set_error(msg);
  return code;
}

int check_hip(hipError_t err, const char* what) {
  if (err == hipSuccess) return MDL_OK;
  return fail(MDL_ERR_HIP, std::string(what) + ": " + hipGetErrorString(err));
}

// ------------------------------------------------------------ bucketing --

// Bucket of one raw value (0 for a null).  mod_magic = ceil(2^64 / m) for
// the mod rule's m = num_buckets - 1 >= 2.
__device__ __forceinline__ int64_t bucket_of(int64_t v, bool present, int64_t num_buckets, int32_t mode,
                                             int32_t validate_nonzero, uint64_t mod_magic, int& bad) {
  if (!present) return 0;
  if (mode == MDL_BUCKET_NONE) return v;
  if (mode == MDL_BUCKET_PRE_HASHED) {
    // Unsigned low bits of the signed hash: identical to the signed modulo
    // for a power-of-two bucket count, INT64_MIN included.
    bad += (validate_nonzero && v == 0);
    return (int64_t)(((uint64_t)v & (uint64_t)(num_buckets - 1)) + 1u);
  }
  // 1 + floormod(v - 1, m) without forming v - 1 or dividing: the sign goes
  // first (x = v or ~v = -v - 1, both below 2^63, INT64_MIN included), and
  // mulhi(x, ceil(2^64 / m)) is floor(x / m) or one more, which one add of m
  // corrects.
  const uint64_t m = (uint64_t)(num_buckets - 1);
  uint64_t fm1 = 0;  // floormod(v - 1, m)
  if (m > 1) {
    const bool neg = v < 0;
    const uint64_t x = neg ? ~(uint64_t)v : (uint64_t)v;
    uint64_t rem = x - __umul64hi(x, mod_magic) * m;
    if ((int64_t)rem < 0) rem += m;
    const uint64_t fm = neg ? m - 1 - rem : rem;  // floormod(v, m)
    fm1 = fm == 0 ? m - 1 : fm - 1;
  }
  return (int64_t)(1 + fm1);
}

__global__ void bucketize_kernel(const int64_t* __restrict__ raw, const uint8_t* __restrict__ valid,
                                 int64_t n, int64_t num_buckets, int32_t mode,
                                 int32_t validate_nonzero, int64_t* __restrict__ out,
                                 int32_t* __restrict__ error_count, uint64_t mod_magic) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  int bad = 0;
  for (; i < n; i += stride) {
    const bool present = valid == nullptr || valid[i] != 0;
    out[i] = bucket_of(raw[i], present, num_buckets, mode, validate_nonzero, mod_magic, bad);
  }
  if (error_count != nullptr && bad) atomicAdd(error_count, bad);
}

static uint64_t mod_magic_for(int32_t mode, int64_t num_buckets) {
  const uint64_t m = (uint64_t)(num_buckets - 1);
  return mode == MDL_BUCKET_MOD && m > 1 ? UINT64_MAX / m + 1 : 0;  // ceil(2^64 / m)
}

static int validate_bucket_mode(const char* who, int32_t mode, int64_t num_buckets) {
  if (mode == MDL_BUCKET_PRE_HASHED) {
    if (num_buckets <= 0 || (num_buckets & (num_buckets - 1)) != 0)
      return fail(MDL_ERR_INVALID, "pre_hashed num_buckets must be a positive power of two");
  } else if (mode == MDL_BUCKET_MOD) {
    if (num_buckets <= 1) return fail(MDL_ERR_INVALID, "mod bucketing needs num_buckets > 1");
  } else {
    return fail(MDL_ERR_INVALID, std::string(who) + ": unknown bucketing mode");
  }
  return MDL_OK;
}

// ------------------------------------------------------ list truncation --

// Kept count and first kept element of every row.  Offsets outside [0, n_in]
// or decreasing are clamped (and counted); a null row keeps nothing.
__global__ void bag_take_kernel(const int64_t* __restrict__ in_offsets, const uint8_t* __restrict__ row_valid,
                                int64_t rows, int64_t n_in, int64_t max_length, int32_t truncation,
                                int64_t* __restrict__ lengths, int64_t* __restrict__ starts,
                                int32_t* __restrict__ error_count) {
  const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= rows) return;
  int64_t lo = in_offsets[r], hi = in_offsets[r + 1];
  int bad = 0;
  if (lo < 0 || lo > n_in) {
    lo = lo < 0 ? 0 : n_in;
    bad = 1;
  }
  if (hi < lo || hi > n_in) {
    hi = hi < lo ? lo : n_in;
    bad = 1;
  }
  int64_t len = hi - lo;
  // A null row keeps nothing, except under tail truncation: the reference
  // rebuilds tail-truncated lists from the raw offsets (src/dataloader.py:
  // 8583-8604), so a null row with a non-empty span keeps its last elements.
  const bool tail_cut = truncation == MDL_TRUNCATE_TAIL && max_length >= 0;
  if (row_valid != nullptr && row_valid[r] == 0 && !tail_cut) len = 0;
  const int64_t take = max_length >= 0 && len > max_length ? max_length : len;
  lengths[r] = take;
  starts[r] = truncation == MDL_TRUNCATE_HEAD ? lo : hi - take;
  if (bad && error_count != nullptr) atomicAdd(error_count, 1);
}

// The row holding kept entry j: the last r in [lo, hi] with off[r] <= j.
__device__ __forceinline__ int64_t row_of(const int64_t* off, int64_t lo, int64_t hi, int64_t j) {
  while (lo < hi) {
    const int64_t mid = (lo + hi + 1) >> 1;
    if (off[mid] <= j) lo = mid;
    else hi = mid - 1;
  }
  return lo;
}

constexpr int kGatherThreads = 256;  // rows per block pass, one thread each to stage them

// Each block pass takes 256 consecutive rows: it stages their kept offsets
// and first source elements in LDS (coalesced), then walks their kept
// entries -- one contiguous stretch of the output -- 256 at a time, each
// thread finding its row by a search in LDS.  The grid then zeroes the
// entries past the kept total.
__global__ __launch_bounds__(kGatherThreads) void bag_gather_kernel(
    const int64_t* __restrict__ out_offsets, const int64_t* __restrict__ starts, int64_t rows,
    const int64_t* __restrict__ raw, const uint8_t* __restrict__ elem_valid, int64_t num_buckets, int32_t mode,
    int32_t validate_nonzero, uint64_t mod_magic, int64_t* __restrict__ values, int64_t capacity,
    int32_t* __restrict__ error_count) {
  __shared__ int64_t s_off[kGatherThreads + 1];
  __shared__ int64_t s_start[kGatherThreads];
  const int tid = threadIdx.x;
  int bad = 0;
  for (int64_t r0 = (int64_t)blockIdx.x * kGatherThreads; r0 < rows; r0 += (int64_t)gridDim.x * kGatherThreads) {
    const int nr = rows - r0 < kGatherThreads ? (int)(rows - r0) : kGatherThreads;
    if (tid < nr) {
      s_off[tid] = out_offsets[r0 + tid];
      s_start[tid] = starts[r0 + tid];
    }
    if (tid == 0) s_off[nr] = out_offsets[r0 + nr];
    __syncthreads();
    const int64_t b = s_off[0];
    const int64_t e = s_off[nr] < capacity ? s_off[nr] : capacity;
    for (int64_t j = b + tid; j < e; j += kGatherThreads) {
      const int64_t r = row_of(s_off, 0, nr - 1, j);
      const int64_t src = s_start[r] + (j - s_off[r]);
      const bool present = elem_valid == nullptr || elem_valid[src] != 0;
      values[j] = bucket_of(raw[src], present, num_buckets, mode, validate_nonzero, mod_magic, bad);
    }
    __syncthreads();  // the next pass restages the LDS
  }
  const int64_t total = out_offsets[rows];
  for (int64_t j = total + (int64_t)blockIdx.x * kGatherThreads + tid; j < capacity;
       j += (int64_t)gridDim.x * kGatherThreads)
    values[j] = 0;
  if (error_count != nullptr && bad) atomicAdd(error_count, bad);
}

// ----------------------------------------------------------------- scan --

constexpr int kScanThreads = 256;
constexpr int kScanItems = 8;
constexpr int kScanTile = kScanThreads * kScanItems;

template <typename T>
__device__ T block_exclusive_scan(T v, T* smem, T* total) {
  // smem: kScanThreads entries.
  const int tid = threadIdx.x;
  smem[tid] = v;
  __syncthreads();
  for (int d = 1; d < kScanThreads; d <<= 1) {
    T o = tid >= d ? smem[tid - d] : T(0);
    __syncthreads();
    smem[tid] += o;
    __syncthreads();
  }
  T incl = smem[tid];
  if (total) *total = smem[kScanThreads - 1];
  __syncthreads();
  return incl - v;
}

__global__ void scan_tile_sums(const int64_t* __restrict__ in, int64_t n, int64_t* __restrict__ sums) {
  __shared__ int64_t smem[kScanThreads];
  const int64_t base = (int64_t)blockIdx.x * kScanTile;
  int64_t s = 0;
#pragma unroll
  for (int k = 0; k < kScanItems; ++k) {
    int64_t i = base + (int64_t)k * kScanThreads + threadIdx.x;
    if (i < n) s += in[i];
  }
  int64_t total;
  block_exclusive_scan<int64_t>(s, smem, &total);
  if (threadIdx.x == 0) sums[blockIdx.x] = total;
}

// Exclusive scan of the per-tile sums in place, one block, any count.
__global__ void scan_sums_single(int64_t* __restrict__ sums, int64_t m) {
  __shared__ int64_t smem[kScanThreads];
  int64_t carry = 0;
  for (int64_t base = 0; base < m; base += kScanThreads) {
    int64_t i = base + threadIdx.x;
    int64_t v = i < m ? sums[i] : 0;
    int64_t total;
    int64_t ex = block_exclusive_scan<int64_t>(v, smem, &total);
    if (i < m) sums[i] = carry + ex;
    carry += total;
  }
}

// offsets[i+1] = sum(in[0..i]); offsets[0] = 0.  The tile's prefix is
// sums[b] after scan_sums_single, or, with prefix_self (few tiles), the sum
// of the raw tile sums before it, added up here: one launch fewer.
__global__ void scan_tiles_final(const int64_t* __restrict__ in, int64_t n,
                                 const int64_t* __restrict__ sums, int64_t* __restrict__ offsets,
                                 int prefix_self) {
  __shared__ int64_t smem[kScanThreads];
  int64_t tile_prefix;
  if (prefix_self) {
    int64_t p = 0;
    for (int64_t j = threadIdx.x; j < (int64_t)blockIdx.x; j += kScanThreads) p += sums[j];
    block_exclusive_scan<int64_t>(p, smem, &tile_prefix);
  } else {
    tile_prefix = sums[blockIdx.x];
  }
  const int64_t base = (int64_t)blockIdx.x * kScanTile + (int64_t)threadIdx.x * kScanItems;
  int64_t v[kScanItems];
  int64_t s = 0;
#pragma unroll
  for (int k = 0; k < kScanItems; ++k) {
    int64_t i = base + k;
    v[k] = i < n ? in[i] : 0;
    s += v[k];
  }
  int64_t ex = block_exclusive_scan<int64_t>(s, smem, nullptr) + tile_prefix;
  if (blockIdx.x == 0 && threadIdx.x == 0) offsets[0] = 0;
#pragma unroll
  for (int k = 0; k < kScanItems; ++k) {
    int64_t i = base + k;
    ex += v[k];
    if (i < n) offsets[i + 1] = ex;
  }
}

static __global__ void zero_offset_kernel(int64_t* p) { *p = 0; }

// Tiles whose prefix the final kernel adds up itself.
constexpr int64_t kScanSelfPrefixTiles = 1024;

}  // namespace mdl

using namespace mdl;

extern "C" {

const char* mdl_last_error(void) { return g_last_error.c_str(); }

int32_t mdl_abi_version(void) { return 6; }

int mdl_bucketize(const int64_t* raw, const uint8_t* valid, int64_t n, int64_t num_buckets,
                  int32_t mode, int32_t validate_nonzero, int64_t* out, int32_t* error_count,
                  void* stream) {
  if (n < 0) return fail(MDL_ERR_INVALID, "mdl_bucketize: negative n");
  int rc = validate_bucket_mode("mdl_bucketize", mode, num_buckets);
  if (rc) return rc;
  if (n == 0) return MDL_OK;
  if (raw == nullptr || out == nullptr) return fail(MDL_ERR_INVALID, "mdl_bucketize: null pointer");
  int64_t blocks = (n + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL(bucketize_kernel, dim3((unsigned)blocks), dim3(256), 0, as_stream(stream), raw,
                     valid, n, num_buckets, mode, validate_nonzero, out, error_count,
                     mod_magic_for(mode, num_buckets));
  MDL_CHECK_LAUNCH("bucketize_kernel");
  return MDL_OK;
}

size_t mdl_bag_truncate_workspace_bytes(int64_t rows) {
  const size_t scan = (mdl_offsets_workspace_bytes(rows) + 255) & ~size_t(255);
  return scan + (size_t)(rows > 0 ? rows : 1) * sizeof(int64_t);
}

int mdl_bag_truncate(const int64_t* in_offsets, const uint8_t* row_valid, int64_t rows, const int64_t* raw,
                     const uint8_t* elem_valid, int64_t n_in, int64_t max_length, int32_t truncation,
                     int32_t bucket_mode, int64_t num_buckets, int32_t validate_nonzero, int64_t* lengths,
                     int64_t* out_offsets, int64_t* values, int64_t values_capacity, int32_t* error_count,
                     void* workspace, size_t workspace_bytes, void* stream) {
  if (rows < 0 || n_in < 0 || values_capacity < 0)
    return fail(MDL_ERR_INVALID, "mdl_bag_truncate: negative count");
  if (truncation != MDL_TRUNCATE_HEAD && truncation != MDL_TRUNCATE_TAIL)
    return fail(MDL_ERR_INVALID, "mdl_bag_truncate: truncation must be head or tail");
  if (bucket_mode != MDL_BUCKET_NONE) {
    int rc = validate_bucket_mode("mdl_bag_truncate", bucket_mode, num_buckets);
    if (rc) return rc;
  }
  if (out_offsets == nullptr || (rows > 0 && (in_offsets == nullptr || lengths == nullptr)) ||
      (values_capacity > 0 && values == nullptr) || (values_capacity > 0 && n_in > 0 && raw == nullptr))
    return fail(MDL_ERR_INVALID, "mdl_bag_truncate: null pointer");
  if (workspace_bytes < mdl_bag_truncate_workspace_bytes(rows) || workspace == nullptr)
    return fail(MDL_ERR_WORKSPACE, "mdl_bag_truncate: workspace too small");
  hipStream_t s = as_stream(stream);
  const size_t scan_bytes = (mdl_offsets_workspace_bytes(rows) + 255) & ~size_t(255);
  int64_t* starts = reinterpret_cast<int64_t*>(static_cast<char*>(workspace) + scan_bytes);
  if (rows > 0) {
    hipLaunchKernelGGL(bag_take_kernel, dim3((unsigned)((rows + 255) / 256)), dim3(256), 0, s, in_offsets,
                       row_valid, rows, n_in, max_length, truncation, lengths, starts, error_count);
    MDL_CHECK_LAUNCH("bag_take_kernel");
  }
  int rc = mdl_lengths_to_offsets(lengths, rows, out_offsets, workspace, scan_bytes, stream);
  if (rc) return rc;
  if (values_capacity == 0) return MDL_OK;
  int64_t blocks = (rows + kGatherThreads - 1) / kGatherThreads;
  if (blocks < 256) blocks = 256;  // the zero fill past the kept total needs a grid of its own size
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL(bag_gather_kernel, dim3((unsigned)blocks), dim3(kGatherThreads), 0, s, out_offsets, starts,
                     rows, raw,
                     elem_valid, num_buckets, bucket_mode, validate_nonzero, mod_magic_for(bucket_mode, num_buckets),
                     values, values_capacity, error_count);
  MDL_CHECK_LAUNCH("bag_gather_kernel");
  return MDL_OK;
}

size_t mdl_offsets_workspace_bytes(int64_t n) {
  int64_t tiles = (n + kScanTile - 1) / kScanTile;
  return (size_t)(tiles + 1) * sizeof(int64_t);
}

int mdl_lengths_to_offsets(const int64_t* lengths, int64_t n, int64_t* offsets, void* workspace,
                           size_t workspace_bytes, void* stream) {
  if (n < 0) return fail(MDL_ERR_INVALID, "mdl_lengths_to_offsets: negative n");
  hipStream_t s = as_stream(stream);
  if (n == 0) {
    // a kernel, not a memset: callers may capture this call in a graph
    hipLaunchKernelGGL(zero_offset_kernel, dim3(1), dim3(1), 0, s, offsets);
    MDL_CHECK_LAUNCH("zero_offset_kernel");
    return MDL_OK;
  }
  if (workspace_bytes < mdl_offsets_workspace_bytes(n))
    return fail(MDL_ERR_WORKSPACE, "mdl_lengths_to_offsets: workspace too small");
  int64_t tiles = (n + kScanTile - 1) / kScanTile;
  int64_t* sums = static_cast<int64_t*>(workspace);
  hipLaunchKernelGGL(scan_tile_sums, dim3((unsigned)tiles), dim3(kScanThreads), 0, s, lengths, n, sums);
  MDL_CHECK_LAUNCH("scan_tile_sums");
  const int self = tiles <= kScanSelfPrefixTiles ? 1 : 0;
  if (!self) {
    hipLaunchKernelGGL(scan_sums_single, dim3(1), dim3(kScanThreads), 0, s, sums, tiles);
    MDL_CHECK_LAUNCH("scan_sums_single");
  }
  hipLaunchKernelGGL(scan_tiles_final, dim3((unsigned)tiles), dim3(kScanThreads), 0, s, lengths, n,
                     sums, offsets, self);
  MDL_CHECK_LAUNCH("scan_tiles_final");
  return MDL_OK;
}

}  // extern "C"
