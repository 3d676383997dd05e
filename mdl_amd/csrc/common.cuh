// Device-side helpers shared by the gfx950 kernels of libmdl_hip.so.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string>

#include "../../include/mdl_hip.h"

namespace mdl {

constexpr int kWave = 64;

typedef uint16_t bf16_t;

// ------------------------------------------------------------ error state --

void set_error(const std::string& msg);
int fail(int code, const std::string& msg);
int check_hip(hipError_t err, const char* what);

#define MDL_CHECK_LAUNCH(what)                                   \
  do {                                                           \
    hipError_t _e = hipGetLastError();                           \
    if (_e != hipSuccess) return ::mdl::check_hip(_e, what);     \
  } while (0)

static inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// ------------------------------------------------------------- numerics --

// fp32 -> bf16, round to nearest even; NaN stays NaN (quiet).  Same rounding
// as torch's Tensor.to(torch.bfloat16).
__device__ __forceinline__ bf16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (bf16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (bf16_t)(u >> 16);
}

__device__ __forceinline__ float bf16_to_f32(bf16_t h) {
  return __uint_as_float(((uint32_t)h) << 16);
}

// ------------------------------------------------------------ vector I/O --
//
// A lane moves C consecutive elements of one row.  For C > 1 the address is
// 16-byte aligned for the weight type (C = 16 / sizeof(T)); C == 1 is the
// scalar path for rows whose byte size or base is not 16-byte aligned.

template <typename T, int C>
struct RowIO;

template <>
struct RowIO<float, 4> {
  static __device__ __forceinline__ void load(const float* p, float (&v)[4]) {
    float4 x = *reinterpret_cast<const float4*>(p);
    v[0] = x.x; v[1] = x.y; v[2] = x.z; v[3] = x.w;
  }
  static __device__ __forceinline__ void store(float* p, const float (&v)[4]) {
    *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
  }
};

template <>
struct RowIO<float, 8> {
  static __device__ __forceinline__ void load(const float* p, float (&v)[8]) {
    float4 x = *reinterpret_cast<const float4*>(p);
    float4 y = *reinterpret_cast<const float4*>(p + 4);
    v[0] = x.x; v[1] = x.y; v[2] = x.z; v[3] = x.w;
    v[4] = y.x; v[5] = y.y; v[6] = y.z; v[7] = y.w;
  }
  static __device__ __forceinline__ void store(float* p, const float (&v)[8]) {
    *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
    *reinterpret_cast<float4*>(p + 4) = make_float4(v[4], v[5], v[6], v[7]);
  }
};

template <>
struct RowIO<bf16_t, 8> {
  static __device__ __forceinline__ void load(const bf16_t* p, float (&v)[8]) {
    uint4 x = *reinterpret_cast<const uint4*>(p);
    uint32_t w[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = __uint_as_float(w[i] << 16);
      v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
  }
  static __device__ __forceinline__ void store(bf16_t* p, const float (&v)[8]) {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      w[i] = (uint32_t)f32_to_bf16(v[2 * i]) | ((uint32_t)f32_to_bf16(v[2 * i + 1]) << 16);
    *reinterpret_cast<uint4*>(p) = make_uint4(w[0], w[1], w[2], w[3]);
  }
};

template <>
struct RowIO<float, 1> {
  static __device__ __forceinline__ void load(const float* p, float (&v)[1]) { v[0] = *p; }
  static __device__ __forceinline__ void store(float* p, const float (&v)[1]) { *p = v[0]; }
};

template <>
struct RowIO<bf16_t, 1> {
  static __device__ __forceinline__ void load(const bf16_t* p, float (&v)[1]) {
    v[0] = bf16_to_f32(*p);
  }
  static __device__ __forceinline__ void store(bf16_t* p, const float (&v)[1]) {
    *p = f32_to_bf16(v[0]);
  }
};

// A row of zeros in device memory.  Lanes whose row is absent (past the end
// of a chunk, an invalid id, a column past dim) load from here instead of
// branching around the load, so every load of a pass issues back to back.
// (One copy per translation unit; only device code reads it.)
static __device__ __align__(256) float g_zero_row[512];

template <typename T>
__device__ __forceinline__ const T* zero_row() {
  return reinterpret_cast<const T*>(g_zero_row);
}

// Rows one pass covers and the chunk length that gives a wave about
// kPassesPerChunk passes.
constexpr int kPassesPerChunk = 32;

// ------------------------------------------------------- row-access classes --
//
// Weight dtype x output/gradient dtype x 16-byte vectors or scalars.  Every
// kernel that moves rows is instantiated once per class and launched only
// for the classes present, so one launch never carries the registers of six
// code paths.

template <typename TW, typename TO, int C>
struct ClassOf;
template <> struct ClassOf<float, float, 4> { static constexpr int value = MDL_CLASS_F32_VEC; };
template <> struct ClassOf<float, float, 1> { static constexpr int value = MDL_CLASS_F32; };
template <> struct ClassOf<bf16_t, bf16_t, 8> { static constexpr int value = MDL_CLASS_BF16_VEC; };
template <> struct ClassOf<bf16_t, bf16_t, 1> { static constexpr int value = MDL_CLASS_BF16; };
template <> struct ClassOf<bf16_t, float, 8> { static constexpr int value = MDL_CLASS_BF16_F32_VEC; };
template <> struct ClassOf<bf16_t, float, 1> { static constexpr int value = MDL_CLASS_BF16_F32; };

__host__ __device__ __forceinline__ int row_class(int wdtype, int odtype, bool vec) {
  const int base = wdtype == MDL_F32 ? MDL_CLASS_F32_VEC
                   : (odtype == MDL_BF16 ? MDL_CLASS_BF16_VEC : MDL_CLASS_BF16_F32_VEC);
  return base + (vec ? 0 : 1);
}

// Whether a feature's weight, output and gradient rows allow 16-byte lanes.
__host__ __device__ __forceinline__ bool feature_vec(uint64_t weight, uint64_t out, int64_t dim,
                                                     int64_t out_stride, int wdtype, int odtype) {
  const int wsz = wdtype == MDL_BF16 ? 2 : 4;
  const int osz = odtype == MDL_BF16 ? 2 : 4;
  const int c = 16 / wsz;
  return weight % 16 == 0 && out % 16 == 0 && (dim * wsz) % 16 == 0 && (out_stride * osz) % 16 == 0 &&
         ((int64_t)c * osz) % 16 == 0;
}

// Whether a table's rows (and its gradient/value rows, laid out alike by
// the caller) allow 16-byte lanes.
__host__ __device__ __forceinline__ bool table_vec_of(uint64_t weight, int64_t dim, int wdtype) {
  const int wsz = wdtype == MDL_BF16 ? 2 : 4;
  return weight % 16 == 0 && (dim * wsz) % 16 == 0;
}

// ------------------------------------------------------------ wave helpers --

__device__ __forceinline__ int lane_id() { return (int)(threadIdx.x & (kWave - 1)); }

__device__ __forceinline__ float shfl_f(float v, int src) {
  return __int_as_float(__builtin_amdgcn_ds_bpermute(src << 2, __float_as_int(v)));
}
__device__ __forceinline__ int shfl_i(int v, int src) {
  return __builtin_amdgcn_ds_bpermute(src << 2, v);
}
__device__ __forceinline__ uint32_t shfl_u(uint32_t v, int src) {
  return (uint32_t)__builtin_amdgcn_ds_bpermute(src << 2, (int)v);
}

// Lanes per row: next power of two >= ceil(dim / C), capped at one wave.
__host__ __device__ __forceinline__ int lanes_for(int dim, int c) {
  int need = (dim + c - 1) / c;
  int l = 1;
  while (l < need && l < kWave) l <<= 1;
  return l;
}

// Remap a linear block index so that each of the 8 XCDs (which receive
// blocks round-robin) works on one contiguous range of the logical index
// space; neighbouring chunks then share that XCD's L2.
__device__ __forceinline__ int64_t xcd_block(int64_t bid, int64_t nblocks) {
  const int64_t kXcd = 8;
  if (nblocks < kXcd * 2) return bid;
  int64_t per = nblocks / kXcd;   // blocks every XCD owns in the regular part
  int64_t regular = per * kXcd;
  if (bid >= regular) return bid;  // tail keeps its position
  return (bid % kXcd) * per + bid / kXcd;
}

}  // namespace mdl
