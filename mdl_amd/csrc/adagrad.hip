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

}  // extern "C"
