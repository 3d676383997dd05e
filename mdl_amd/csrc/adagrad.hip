// Row-wise Adagrad on the unique rows of one table.
//
// L lanes own one row (16 bytes each), so a wavefront updates 64/L rows per
// pass with one read and one write of every touched weight row, its gradient
// row and its fp32 accumulator; a row wider than 64 lanes cover is walked in
// column blocks by one wave (any dim, like the reference kernel's
// BLOCK = next_pow2(dim)).  The row's sum of squares is combined across
// its L lanes with cross-lane permutes; the arithmetic follows the reference
// update kernel (mean of squares, sqrt, eps added after the root, division
// before the learning-rate product, one rounding to the weight dtype).
#include "common.cuh"

namespace mdl {

constexpr int kAdaWaves = 4;
constexpr int kAdaUnroll = 2;

struct AdaArgs {
  void* weight;
  int64_t num_rows;
  int64_t wstride;
  float* acc;
  const int64_t* rows;
  int64_t n;
  const void* values;
  int64_t vstride;
  int32_t dim;
  float lr, eps;
  int32_t* error_count;
};

template <typename TW, typename TV, int C>
__device__ __forceinline__ void adagrad_rows(const AdaArgs& a, int64_t wave, int64_t nwaves) {
  const int lane = lane_id();
  const int L = lanes_for(a.dim, C);
  const int G = kWave / L;
  const int slot = lane / L, sub = lane % L;
  const int col = sub * C;
  const bool col_ok = col < a.dim;
  TW* W = static_cast<TW*>(a.weight);
  const TV* V = static_cast<const TV*>(a.values);
  int bad = 0;
  for (int64_t base = wave * G * kAdaUnroll; base < a.n; base += nwaves * G * kAdaUnroll) {
    float g[kAdaUnroll][C], w[kAdaUnroll][C];
    int64_t row[kAdaUnroll];
    bool ok[kAdaUnroll];
#pragma unroll
    for (int u = 0; u < kAdaUnroll; ++u) {
      const int64_t i = base + u * G + slot;
      const bool valid = i < a.n;
      row[u] = valid ? a.rows[i] : 0;
      ok[u] = valid && (uint64_t)row[u] < (uint64_t)a.num_rows;
      if (valid && !ok[u] && sub == 0) ++bad;
#pragma unroll
      for (int k = 0; k < C; ++k) g[u][k] = w[u][k] = 0.f;
      if (ok[u] && col_ok) {
        RowIO<TV, C>::load(V + i * a.vstride + col, g[u]);
        RowIO<TW, C>::load(W + row[u] * a.wstride + col, w[u]);
      }
    }
#pragma unroll
    for (int u = 0; u < kAdaUnroll; ++u) {
      float ss = 0.f;
#pragma unroll
      for (int k = 0; k < C; ++k) ss += g[u][k] * g[u][k];
      for (int m = 1; m < L; m <<= 1) ss += shfl_f(ss, lane ^ m);
      if (ok[u]) {
        const float acc = a.acc[row[u]] + ss / (float)a.dim;
        if (sub == 0) a.acc[row[u]] = acc;
        const float den = sqrtf(acc) + a.eps;
        if (col_ok) {
#pragma unroll
          for (int k = 0; k < C; ++k) w[u][k] = w[u][k] - a.lr * (g[u][k] / den);
          RowIO<TW, C>::store(W + row[u] * a.wstride + col, w[u]);
        }
      }
    }
  }
  if (bad && a.error_count) atomicAdd(a.error_count, bad);
}

// Rows wider than one wavefront covers (dim > 64 * C): the wave owns one row
// at a time and walks it in column blocks of 64 * C elements, twice -- the
// first walk adds up the row's sum of squares, the second (after the
// accumulator update, which needs the whole row's mean square) reads the
// gradient again with the weight and writes the updated weight.  The second
// read of the gradient row mostly hits the cache.
template <typename TW, typename TV, int C>
__device__ __forceinline__ void adagrad_wide_rows(const AdaArgs& a, int64_t wave, int64_t nwaves) {
  const int lane = lane_id();
  const int span = kWave * C;
  const int ncb = (a.dim + span - 1) / span;
  TW* W = static_cast<TW*>(a.weight);
  const TV* V = static_cast<const TV*>(a.values);
  int bad = 0;
  for (int64_t i = wave; i < a.n; i += nwaves) {
    const int64_t row = a.rows[i];
    if ((uint64_t)row >= (uint64_t)a.num_rows) {
      if (lane == 0) ++bad;
      continue;
    }
    const TV* vrow = V + i * a.vstride;
    TW* wrow = W + row * a.wstride;
    float ss = 0.f;
    for (int cb = 0; cb < ncb; ++cb) {
      const int col = cb * span + lane * C;
      if (col < a.dim) {
        float g[C];
        RowIO<TV, C>::load(vrow + col, g);
#pragma unroll
        for (int k = 0; k < C; ++k) ss += g[k] * g[k];
      }
    }
    for (int m = 1; m < kWave; m <<= 1) ss += shfl_f(ss, lane ^ m);
    const float acc = a.acc[row] + ss / (float)a.dim;
    if (lane == 0) a.acc[row] = acc;
    const float den = sqrtf(acc) + a.eps;
    for (int cb = 0; cb < ncb; ++cb) {
      const int col = cb * span + lane * C;
      if (col < a.dim) {
        float g[C], w[C];
        RowIO<TV, C>::load(vrow + col, g);
        RowIO<TW, C>::load(wrow + col, w);
#pragma unroll
        for (int k = 0; k < C; ++k) w[k] = w[k] - a.lr * (g[k] / den);
        RowIO<TW, C>::store(wrow + col, w);
      }
    }
  }
  if (bad && a.error_count) atomicAdd(a.error_count, bad);
}

template <typename TW, typename TV, int C>
__global__ __launch_bounds__(kAdaWaves * kWave) void adagrad_kernel(AdaArgs a) {
  const int64_t nwaves = (int64_t)gridDim.x * kAdaWaves;
  const int64_t wave = (int64_t)blockIdx.x * kAdaWaves + threadIdx.x / kWave;
  if (a.dim > kWave * C) adagrad_wide_rows<TW, TV, C>(a, wave, nwaves);
  else adagrad_rows<TW, TV, C>(a, wave, nwaves);
}

// ------------------------------------------------------------ grouped --
//
// Every table of an optimizer step in one launch (src/optim.py:299-377 makes
// one update launch per parameter).  The work is cut into units of
// MDL_UPDATE_UNIT entries of one table, one wave each; a table's first unit is
// in its descriptor, and a wave finds its table by binary search over them.
// Entries at or past a table's device-side count (rows present this step)
// are skipped, so a capacity-sized gradient needs no host round trip.

struct GroupedArgs {
  const mdl_update* ups;
  int32_t num;
  int64_t units;
  float eps;
  int32_t* error_count;
};

__host__ __device__ __forceinline__ bool update_vec(const mdl_update& u) {
  const int wsz = u.wdtype == MDL_BF16 ? 2 : 4;
  const int vsz = u.vdtype == MDL_BF16 ? 2 : 4;
  const int c = 16 / wsz;
  return u.weight % 16 == 0 && u.values % 16 == 0 && (u.weight_stride * wsz) % 16 == 0 &&
         (u.values_stride * vsz) % 16 == 0 && ((int64_t)u.dim * wsz) % 16 == 0 && ((int64_t)c * vsz) % 16 == 0;
}

__host__ __device__ __forceinline__ int update_class(int wdtype, int vdtype, bool vec) {
  const int base = wdtype == MDL_F32 ? MDL_CLASS_F32_VEC
                   : (vdtype == MDL_BF16 ? MDL_CLASS_BF16_VEC : MDL_CLASS_BF16_F32_VEC);
  return base + (vec ? 0 : 1);
}

template <typename TW, typename TV, bool kVec>
__global__ __launch_bounds__(kAdaWaves * kWave) void grouped_adagrad_kernel(GroupedArgs g) {
  constexpr int C = kVec ? 16 / (int)sizeof(TW) : 1;
  const int64_t unit = (int64_t)blockIdx.x * kAdaWaves + threadIdx.x / kWave;
  if (unit >= g.units) return;
  int lo = 0, hi = g.num - 1;  // last table whose first unit <= unit
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (g.ups[mid].unit_first <= unit) lo = mid;
    else hi = mid - 1;
  }
  const mdl_update& u = g.ups[lo];
  if (update_class(u.wdtype, u.vdtype, update_vec(u)) != ClassOf<TW, TV, kVec>::value) return;
  int64_t present = u.count != 0 ? *reinterpret_cast<const int64_t*>(u.count) : u.capacity;
  present = present < 0 ? 0 : (present > u.capacity ? u.capacity : present);
  const int64_t start = (unit - u.unit_first) * MDL_UPDATE_UNIT;
  if (start >= present) return;
  AdaArgs a;
  a.weight = reinterpret_cast<void*>(u.weight);
  a.num_rows = u.num_rows;
  a.wstride = u.weight_stride;
  a.acc = reinterpret_cast<float*>(u.state);
  a.rows = reinterpret_cast<const int64_t*>(u.rows) + start;
  a.n = present - start < MDL_UPDATE_UNIT ? present - start : MDL_UPDATE_UNIT;
  a.values = reinterpret_cast<const TV*>(u.values) + start * u.values_stride;
  a.vstride = u.values_stride;
  a.dim = u.dim;
  a.lr = u.lr;
  a.eps = g.eps;
  a.error_count = g.error_count;
  if (a.dim > kWave * C) adagrad_wide_rows<TW, TV, C>(a, 0, 1);
  else adagrad_rows<TW, TV, C>(a, 0, 1);
}

struct LaunchGrouped {
  const GroupedArgs& g;
  int64_t blocks;
  hipStream_t s;
  template <typename TW, typename TV, bool kVec>
  int operator()() const {
    hipLaunchKernelGGL((grouped_adagrad_kernel<TW, TV, kVec>), dim3((unsigned)blocks), dim3(kAdaWaves * kWave), 0,
                       s, g);
    MDL_CHECK_LAUNCH("grouped_adagrad_kernel");
    return MDL_OK;
  }
};

}  // namespace mdl

using namespace mdl;

extern "C" {

int mdl_rowwise_adagrad(void* weight, int32_t wdtype, int64_t num_rows, int32_t dim, int64_t weight_stride,
                        float* acc, const int64_t* rows, int64_t num_touched, const void* values, int32_t vdtype,
                        int64_t values_stride, float lr, float eps, int32_t* error_count, void* stream) {
  if (num_touched < 0 || dim <= 0 || num_rows < 0) return fail(MDL_ERR_INVALID, "mdl_rowwise_adagrad: bad sizes");
  if (num_touched == 0) return MDL_OK;
  if (!weight || !acc || !rows || !values) return fail(MDL_ERR_INVALID, "mdl_rowwise_adagrad: null pointer");
  if (wdtype == MDL_F32 && vdtype != MDL_F32)
    return fail(MDL_ERR_UNSUPPORTED, "mdl_rowwise_adagrad: fp32 weights need fp32 values");
  AdaArgs a;
  a.weight = weight;
  a.num_rows = num_rows;
  a.wstride = weight_stride;
  a.acc = acc;
  a.rows = rows;
  a.n = num_touched;
  a.values = values;
  a.vstride = values_stride;
  a.dim = dim;
  a.lr = lr;
  a.eps = eps;
  a.error_count = error_count;
  const int wsz = wdtype == MDL_BF16 ? 2 : 4;
  const int vsz = vdtype == MDL_BF16 ? 2 : 4;
  const int c = 16 / wsz;
  const bool vec = ((uint64_t)weight % 16 == 0) && ((uint64_t)values % 16 == 0) &&
                   (weight_stride * wsz) % 16 == 0 && (values_stride * vsz) % 16 == 0 &&
                   ((int64_t)dim * wsz) % 16 == 0 && ((int64_t)c * vsz) % 16 == 0;
  const int cc = vec ? c : 1;
  // Rows wider than 64 * cc take one wave each (column-block walk).
  const int L = lanes_for(dim, cc);
  const int64_t rows_per_block = dim > kWave * cc ? kAdaWaves : (int64_t)(kWave / L) * kAdaUnroll * kAdaWaves;
  int64_t blocks = (num_touched + rows_per_block - 1) / rows_per_block;
  if (blocks > 16384) blocks = 16384;
  hipStream_t s = as_stream(stream);
  dim3 g((unsigned)blocks), b(kAdaWaves * kWave);
  if (wdtype == MDL_F32) {
    if (vec) hipLaunchKernelGGL((adagrad_kernel<float, float, 4>), g, b, 0, s, a);
    else hipLaunchKernelGGL((adagrad_kernel<float, float, 1>), g, b, 0, s, a);
  } else if (vdtype == MDL_BF16) {
    if (vec) hipLaunchKernelGGL((adagrad_kernel<bf16_t, bf16_t, 8>), g, b, 0, s, a);
    else hipLaunchKernelGGL((adagrad_kernel<bf16_t, bf16_t, 1>), g, b, 0, s, a);
  } else {
    if (vec) hipLaunchKernelGGL((adagrad_kernel<bf16_t, float, 8>), g, b, 0, s, a);
    else hipLaunchKernelGGL((adagrad_kernel<bf16_t, float, 1>), g, b, 0, s, a);
  }
  MDL_CHECK_LAUNCH("adagrad_kernel");
  return MDL_OK;
}

uint32_t mdl_update_classes(const mdl_update* updates_host, int32_t num_updates) {
  uint32_t m = 0;
  for (int32_t i = 0; i < num_updates; ++i) {
    const mdl_update& u = updates_host[i];
    m |= 1u << (update_class(u.wdtype, u.vdtype, update_vec(u)) * kWidths);
  }
  return m;
}

int mdl_grouped_rowwise_adagrad(const mdl_update* updates, const mdl_update* updates_host, int32_t num_updates,
                                float eps, int32_t* error_count, void* stream) {
  if (num_updates < 0) return fail(MDL_ERR_INVALID, "mdl_grouped_rowwise_adagrad: negative count");
  if (num_updates == 0) return MDL_OK;
  if (!updates || !updates_host) return fail(MDL_ERR_INVALID, "mdl_grouped_rowwise_adagrad: null pointer");
  int64_t units = 0;
  for (int32_t i = 0; i < num_updates; ++i) {
    const mdl_update& u = updates_host[i];
    if (u.capacity < 0 || u.dim <= 0 || u.num_rows < 0)
      return fail(MDL_ERR_INVALID, "mdl_grouped_rowwise_adagrad: bad sizes");
    if (u.wdtype == MDL_F32 && u.vdtype != MDL_F32)
      return fail(MDL_ERR_UNSUPPORTED, "mdl_grouped_rowwise_adagrad: fp32 weights need fp32 values");
    if (u.unit_first != units)
      return fail(MDL_ERR_INVALID, "mdl_grouped_rowwise_adagrad: unit_first must be the prefix of "
                                   "ceil(capacity / MDL_UPDATE_UNIT)");
    units += (u.capacity + MDL_UPDATE_UNIT - 1) / MDL_UPDATE_UNIT;
  }
  if (units == 0) return MDL_OK;
  GroupedArgs g;
  g.ups = updates;
  g.num = num_updates;
  g.units = units;
  g.eps = eps;
  g.error_count = error_count;
  const int64_t blocks = (units + kAdaWaves - 1) / kAdaWaves;
  if (blocks > 0x7fffffffll) return fail(MDL_ERR_UNSUPPORTED, "mdl_grouped_rowwise_adagrad: too many rows");
  return for_each_class(mdl_update_classes(updates_host, num_updates), LaunchGrouped{g, blocks, as_stream(stream)});
}

}  // extern "C"
