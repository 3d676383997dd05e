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

// mod_magic = ceil(2^64 / m) for the mod rule's m = num_buckets - 1 >= 2.
__global__ void bucketize_kernel(const int64_t* __restrict__ raw, const uint8_t* __restrict__ valid,
                                 int64_t n, int64_t num_buckets, int32_t mode,
                                 int32_t validate_nonzero, int64_t* __restrict__ out,
                                 int32_t* __restrict__ error_count, uint64_t mod_magic) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  int bad = 0;
  for (; i < n; i += stride) {
    const int64_t v = raw[i];
    const bool present = valid == nullptr || valid[i] != 0;
    int64_t r = 0;
    if (present) {
      if (mode == MDL_BUCKET_PRE_HASHED) {
        // Unsigned low bits of the signed hash: identical to the signed
        // modulo for a power-of-two bucket count, INT64_MIN included.
        r = (int64_t)(((uint64_t)v & (uint64_t)(num_buckets - 1)) + 1u);
        bad += (validate_nonzero && v == 0);
      } else {
        // 1 + floormod(v - 1, m) without forming v - 1 or dividing: the sign
        // goes first (x = v or ~v = -v - 1, both below 2^63, INT64_MIN
        // included), and mulhi(x, ceil(2^64 / m)) is floor(x / m) or one
        // more, which one add of m corrects.
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
        r = (int64_t)(1 + fm1);
      }
    }
    out[i] = r;
  }
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

int32_t mdl_abi_version(void) { return 5; }

int mdl_bucketize(const int64_t* raw, const uint8_t* valid, int64_t n, int64_t num_buckets,
                  int32_t mode, int32_t validate_nonzero, int64_t* out, int32_t* error_count,
                  void* stream) {
  if (n < 0) return fail(MDL_ERR_INVALID, "mdl_bucketize: negative n");
  if (mode == MDL_BUCKET_PRE_HASHED) {
    if (num_buckets <= 0 || (num_buckets & (num_buckets - 1)) != 0)
      return fail(MDL_ERR_INVALID, "pre_hashed num_buckets must be a positive power of two");
  } else if (mode == MDL_BUCKET_MOD) {
    if (num_buckets <= 1) return fail(MDL_ERR_INVALID, "mod bucketing needs num_buckets > 1");
  } else {
    return fail(MDL_ERR_INVALID, "mdl_bucketize: unknown mode");
  }
  if (n == 0) return MDL_OK;
  if (raw == nullptr || out == nullptr) return fail(MDL_ERR_INVALID, "mdl_bucketize: null pointer");
  int64_t blocks = (n + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  const uint64_t m = (uint64_t)(num_buckets - 1);
  const uint64_t mod_magic = mode == MDL_BUCKET_MOD && m > 1 ? UINT64_MAX / m + 1 : 0;  // ceil(2^64 / m)
  hipLaunchKernelGGL(bucketize_kernel, dim3((unsigned)blocks), dim3(256), 0, as_stream(stream), raw,
                     valid, n, num_buckets, mode, validate_nonzero, out, error_count, mod_magic);
  MDL_CHECK_LAUNCH("bucketize_kernel");
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
