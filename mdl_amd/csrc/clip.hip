// Global L2-norm clipping of gradients (the sparse clip of the trainer,
// src/train.py:5745-5826): one multi-tensor sum of squares, the clip
// coefficient computed on the device, and one multi-tensor in-place scale.
//
// The sum of squares is deterministic: every span is cut into the same
// kNormParts block-slices whatever the scheduling, each block reduces its
// slice in a fixed tree order, and one block adds the per-slice partials in
// slice order in fp64.  The scale is an HBM-bound elementwise pass with
// 16-byte accesses where the span is aligned.
#include "common.cuh"

namespace mdl {

constexpr int kNormThreads = 256;
constexpr int kNormParts = 128;  // block-slices per span

__device__ __forceinline__ float block_sum(float v, float* smem) {
  for (int m = kWave / 2; m >= 1; m >>= 1) v += __shfl_xor(v, m);
  const int w = threadIdx.x / kWave;
  if (lane_id() == 0) smem[w] = v;
  __syncthreads();
  float t = 0.f;
  if (threadIdx.x == 0)
    for (int i = 0; i < kNormThreads / kWave; ++i) t += smem[i];
  return t;
}

// The span's element count: all numel, or its live rows' elements.
__device__ __forceinline__ int64_t span_elems(const mdl_span& s) {
  if (!s.live_rows) return s.numel;
  const int64_t live = *s.live_rows * (int64_t)s.row_elems;
  return live < 0 ? 0 : (live < s.numel ? live : s.numel);
}

// Elements [lo, hi) of a span, as this block's slice.
__device__ __forceinline__ void slice_of(int64_t n, int64_t* lo, int64_t* hi) {
  const int64_t per = ((n + kNormParts - 1) / kNormParts + 7) & ~int64_t(7);
  *lo = (int64_t)blockIdx.x * per;
  *hi = *lo + per < n ? *lo + per : n;
  if (*hi < *lo) *hi = *lo;  // slices past the end are empty
}

__global__ __launch_bounds__(kNormThreads) void span_sumsq_kernel(const mdl_span* __restrict__ spans,
                                                                   float* __restrict__ partial) {
  __shared__ float smem[kNormThreads / kWave];
  const mdl_span s = spans[blockIdx.y];
  int64_t lo, hi;
  slice_of(span_elems(s), &lo, &hi);
  float acc = 0.f;
  if (s.dtype == MDL_F32) {
    const float* p = reinterpret_cast<const float*>(s.data);
    if (s.data % 16 == 0) {
      // lo is a multiple of 8, so p + lo stays 16-byte aligned
      const int64_t nv = (hi - lo) / 4;
      for (int64_t i = threadIdx.x; i < nv; i += kNormThreads) {
        float v[4];
        RowIO<float, 4>::load(p + lo + 4 * i, v);
        acc += v[0] * v[0] + v[1] * v[1] + v[2] * v[2] + v[3] * v[3];
      }
      for (int64_t i = lo + 4 * nv + threadIdx.x; i < hi; i += kNormThreads) acc += p[i] * p[i];
    } else {
      for (int64_t i = lo + threadIdx.x; i < hi; i += kNormThreads) acc += p[i] * p[i];
    }
  } else {
    const bf16_t* p = reinterpret_cast<const bf16_t*>(s.data);
    if (s.data % 16 == 0) {
      const int64_t nv = (hi - lo) / 8;
      for (int64_t i = threadIdx.x; i < nv; i += kNormThreads) {
        float v[8];
        RowIO<bf16_t, 8>::load(p + lo + 8 * i, v);
#pragma unroll
        for (int k = 0; k < 8; ++k) acc += v[k] * v[k];
      }
      for (int64_t i = lo + 8 * nv + threadIdx.x; i < hi; i += kNormThreads) {
        const float x = bf16_to_f32(p[i]);
        acc += x * x;
      }
    } else {
      for (int64_t i = lo + threadIdx.x; i < hi; i += kNormThreads) {
        const float x = bf16_to_f32(p[i]);
        acc += x * x;
      }
    }
  }
  const float t = block_sum(acc, smem);
  if (threadIdx.x == 0) partial[(int64_t)blockIdx.y * kNormParts + blockIdx.x] = t;
}

// out[0] = sum of m partials, added in a fixed order in fp64: thread t adds
// partials t, t + kSumThreads, ... in index order (eight loads issued before
// their additions), then a fixed tree joins the threads.  One block of 1024
// threads: the per-chunk partials of a c1 backward (17-42 K of them) take
// about five memory round trips instead of twenty (22.6 us with 256 threads).
constexpr int kSumThreads = 1024;
__global__ __launch_bounds__(kSumThreads) void sum_partials_kernel(const float* __restrict__ partial, int64_t m,
                                                                    const int64_t* m_dev, float* out) {
  __shared__ double smem[kSumThreads];
  if (m_dev) m = *m_dev;
  constexpr int kBatch = 8;
  double acc = 0.0;
  for (int64_t base = 0; base < m; base += (int64_t)kSumThreads * kBatch) {
    float v[kBatch];
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
      const int64_t i = base + (int64_t)j * kSumThreads + threadIdx.x;
      v[j] = i < m ? partial[i] : 0.f;
    }
#pragma unroll
    for (int j = 0; j < kBatch; ++j) acc += (double)v[j];
  }
  smem[threadIdx.x] = acc;
  __syncthreads();
  for (int d = kSumThreads / 2; d >= 1; d >>= 1) {
    if (threadIdx.x < d) smem[threadIdx.x] += smem[threadIdx.x + d];
    __syncthreads();
  }
  if (threadIdx.x == 0) out[0] = (float)smem[0];
}

// total = sqrt(sum of the count squared norms), added in fp32 in order like
// the trainer's replicated + sharded sum; coef = min(max_norm / (total + 1e-6), 1).
__global__ void clip_coef_kernel(const float* __restrict__ sumsq, int32_t count, float max_norm, float* total_norm,
                                 float* coef) {
  if (threadIdx.x != 0 || blockIdx.x != 0) return;
  float t = 0.f;
  for (int32_t i = 0; i < count; ++i) t += sumsq[i];
  const float norm = sqrtf(t);
  const float c = max_norm / (norm + 1e-6f);
  if (total_norm) total_norm[0] = norm;
  coef[0] = c < 1.f ? c : 1.f;
}

// x *= coef in the span's dtype: for bf16 the coefficient is rounded to bf16
// first and the product rounded once (torch's bf16 multiply of the
// coefficient cast to the gradient dtype, src/train.py:5756-5772).
__global__ __launch_bounds__(kNormThreads) void span_scale_kernel(const mdl_span* __restrict__ spans,
                                                                   const float* __restrict__ coef_p) {
  const mdl_span s = spans[blockIdx.y];
  int64_t lo, hi;
  slice_of(span_elems(s), &lo, &hi);
  const float coef = coef_p[0];
  if (s.dtype == MDL_F32) {
    float* p = reinterpret_cast<float*>(s.data);
    int64_t done = lo;
    if (s.data % 16 == 0) {
      const int64_t nv = (hi - lo) / 4;
      for (int64_t i = threadIdx.x; i < nv; i += kNormThreads) {
        float v[4];
        RowIO<float, 4>::load(p + lo + 4 * i, v);
#pragma unroll
        for (int k = 0; k < 4; ++k) v[k] *= coef;
        RowIO<float, 4>::store(p + lo + 4 * i, v);
      }
      done = lo + 4 * nv;
    }
    for (int64_t i = done + threadIdx.x; i < hi; i += kNormThreads) p[i] *= coef;
  } else {
    const float cb = bf16_to_f32(f32_to_bf16(coef));
    bf16_t* p = reinterpret_cast<bf16_t*>(s.data);
    int64_t done = lo;
    if (s.data % 16 == 0) {
      const int64_t nv = (hi - lo) / 8;
      for (int64_t i = threadIdx.x; i < nv; i += kNormThreads) {
        float v[8];
        RowIO<bf16_t, 8>::load(p + lo + 8 * i, v);
#pragma unroll
        for (int k = 0; k < 8; ++k) v[k] *= cb;
        RowIO<bf16_t, 8>::store(p + lo + 8 * i, v);
      }
      done = lo + 8 * nv;
    }
    for (int64_t i = done + threadIdx.x; i < hi; i += kNormThreads) p[i] = f32_to_bf16(bf16_to_f32(p[i]) * cb);
  }
}

int launch_sum_partials(const float* partial, int64_t m, const int64_t* m_dev, float* out, hipStream_t s) {
  hipLaunchKernelGGL(sum_partials_kernel, dim3(1), dim3(kSumThreads), 0, s, partial, m, m_dev, out);
  MDL_CHECK_LAUNCH("sum_partials_kernel");
  return MDL_OK;
}

}  // namespace mdl

using namespace mdl;

extern "C" {

size_t mdl_sumsq_workspace_bytes(int32_t num_spans) {
  return (size_t)(num_spans > 0 ? num_spans : 1) * kNormParts * sizeof(float) + 256;
}

int mdl_sumsq(const mdl_span* spans, int32_t num_spans, float* sumsq, void* workspace, size_t workspace_bytes,
              void* stream) {
  if (num_spans < 0 || num_spans > 65535) return fail(MDL_ERR_INVALID, "mdl_sumsq: num_spans outside [0, 65535]");
  if (!sumsq) return fail(MDL_ERR_INVALID, "mdl_sumsq: null output");
  if (workspace_bytes < mdl_sumsq_workspace_bytes(num_spans))
    return fail(MDL_ERR_WORKSPACE, "mdl_sumsq: workspace too small");
  hipStream_t s = as_stream(stream);
  float* partial = static_cast<float*>(workspace);
  if (num_spans > 0) {
    if (!spans) return fail(MDL_ERR_INVALID, "mdl_sumsq: null spans");
    hipLaunchKernelGGL(span_sumsq_kernel, dim3(kNormParts, (unsigned)num_spans), dim3(kNormThreads), 0, s, spans,
                       partial);
    MDL_CHECK_LAUNCH("span_sumsq_kernel");
  }
  return launch_sum_partials(partial, (int64_t)num_spans * kNormParts, nullptr, sumsq, s);
}

int mdl_clip_coef(const float* sumsq, int32_t count, float max_norm, float* total_norm, float* coef, void* stream) {
  if (count < 0 || (count > 0 && !sumsq) || !coef) return fail(MDL_ERR_INVALID, "mdl_clip_coef: bad arguments");
  hipLaunchKernelGGL(clip_coef_kernel, dim3(1), dim3(kWave), 0, as_stream(stream), sumsq, count, max_norm,
                     total_norm, coef);
  MDL_CHECK_LAUNCH("clip_coef_kernel");
  return MDL_OK;
}

int mdl_scale(const mdl_span* spans, int32_t num_spans, const float* coef, void* stream) {
  if (num_spans < 0 || num_spans > 65535) return fail(MDL_ERR_INVALID, "mdl_scale: num_spans outside [0, 65535]");
  if (num_spans == 0) return MDL_OK;
  if (!spans || !coef) return fail(MDL_ERR_INVALID, "mdl_scale: null pointer");
  hipLaunchKernelGGL(span_scale_kernel, dim3(kNormParts, (unsigned)num_spans), dim3(kNormThreads), 0,
                     as_stream(stream), spans, coef);
  MDL_CHECK_LAUNCH("span_scale_kernel");
  return MDL_OK;
}

}  // extern "C"
