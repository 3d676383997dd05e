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

// Correctly rounded reciprocals 1/d of the small bag weight counts d, folded
// by the compiler (IEEE division at compile time); entry 0 is unused.
constexpr int kRcpTable = 256;
struct RcpTable {
  float v[kRcpTable];
  constexpr RcpTable() : v() {
    v[0] = 1.0f;
    for (int i = 1; i < kRcpTable; ++i) v[i] = 1.0f / (float)i;
  }
};
__device__ constexpr RcpTable kBagRcp{};

// Division by a bag's weight count d (an integer >= 1 held in fp32) with the
// result of a correctly rounded v / d, for one reciprocal per bag instead of
// one division per element: with r = 1/d correctly rounded (from the table
// for d < 256, else one division, in a branch taken only by such lanes),
// q = v * r, the exact residual e = v - q * d (one FMA) corrects q to
// q + e * r (Markstein's correction).  It equals the IEEE quotient for every
// fp32 v whose quotient is a normal number: checked over all 2^23
// significands for every d in [1, 65536] and for 4096 random d up to 2^24
// against x86's correctly rounded division.  d = 1 gives v exactly.
__device__ __noinline__ float bag_rcp_slow(float d) { return 1.0f / d; }

struct BagDivisor {
  float d, r;
  __device__ __forceinline__ explicit BagDivisor(float count) : d(count) {
    const int i = (int)count;
    r = kBagRcp.v[i < kRcpTable ? i : 0];
    if (__builtin_expect(i >= kRcpTable, 0)) r = bag_rcp_slow(count);
  }
  __device__ __forceinline__ float operator()(float v) const {
    const float q = __fmul_rn(v, r);
    return __builtin_fmaf(__builtin_fmaf(-q, d, v), r, q);
  }
};

// ------------------------------------------------------------ vector I/O --
//
// A lane moves C consecutive elements of one row.  For C > 1 the address is
// 16-byte aligned and C is a multiple of one 16-byte vector of the type
// (4 fp32 or 8 bf16), so a lane issues C/4 (fp32) or C/8 (bf16) 16-byte
// accesses; C == 1 is the scalar path for rows whose byte size or base is not
// 16-byte aligned.

// A row of zeros in device memory.  Lanes whose row is absent (past the end
// of a chunk, an invalid id, a column past dim) load from here instead of
// branching around the load, so every load of a pass issues back to back.
// (One copy per translation unit; only device code reads it.)
static __device__ __align__(256) float g_zero_row[512];

template <typename T>
__device__ __forceinline__ const T* zero_row() {
  return reinterpret_cast<const T*>(g_zero_row);
}

template <typename T, int C>
struct RowIO;

// Cache policy of a row access.  kStream marks data a kernel touches once
// (outputs and sort keys written for a later kernel): it is stored with the
// non-temporal hint, so it does not push out of L2 the rows that are read
// again (Zipf-hot weight rows in the lookup).
enum CachePolicy { kKeep = 0, kStream = 1 };

// Which accesses stream (compile-time switches): the lookup's outputs and
// sort keys (on: c1 forward 0.290 -> 0.282 ms, reduce 0.510 -> 0.498 ms), and
// the update's weight rows and accumulators (off: streaming them slowed the
// reduce from 0.51 to 0.54 ms; streaming only their loads 0.536 ms, only the
// weight rows' loads 0.535 ms, only the stores no change).
#ifndef MDL_STREAM_UPDATE
#define MDL_STREAM_UPDATE 0
#endif
#ifndef MDL_STREAM_OUT
#define MDL_STREAM_OUT 1
#endif
constexpr int kUpdatePolicy = MDL_STREAM_UPDATE ? kStream : kKeep;
// Gradient rows in the backward reduce: 0 keep, 1 stream the rows of tables
// read by one unpooled feature (each read once, so L2 keeps the bag rows that
// every id of a bag reads again: c1 apply 0.541 -> 0.535 ms over two paired
// runs, other configs unchanged), 2 stream all (0.54 -> 0.71 ms: the
// re-reads then all miss).
#ifndef MDL_STREAM_GRAD
#define MDL_STREAM_GRAD 1
#endif
constexpr int kOutPolicy = MDL_STREAM_OUT ? kStream : kKeep;

// fp32 rows copied eight elements per lane as two 16-byte pieces, lane sub
// holding pieces sub and sub + L of its slot's row: each load or store
// instruction then covers 16·L contiguous bytes of the row.  Eight
// consecutive elements per lane would make each instruction cover every
// other 16 bytes, and non-temporal stores leave L2 before the two halves of
// a 64-byte segment meet (c1 forward 0.291 -> 0.276 ms, c2 sequence gather
// 0.154 -> 0.139 ms per feature).
#ifndef MDL_SPLIT_ROWS
#define MDL_SPLIT_ROWS 1
#endif

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Every row, id, key and accumulator access goes through a global
// address-space pointer.  Pointers the kernels read out of descriptors are
// generic to the compiler, which would otherwise emit flat instructions for
// them; a flat load also counts against the LDS counter, so each wait for an
// LDS value (staged keys, bag bounds) would wait for every row load in
// flight as well.
template <typename T>
using gptr = __attribute__((address_space(1))) T*;

template <typename T>
__device__ __forceinline__ const gptr<T> to_global(const T* p) {
  return (const gptr<T>)p;
}
template <typename T>
__device__ __forceinline__ gptr<T> to_global(T* p) {
  return (gptr<T>)p;
}

template <int kPolicy = kKeep, typename T>
__device__ __forceinline__ T ld_policy(const T* p) {
  if constexpr (kPolicy == kStream) return __builtin_nontemporal_load(to_global(p));
  else return *to_global(p);
}
template <int kPolicy = kKeep, typename T>
__device__ __forceinline__ void st_policy(T* p, T v) {
  if constexpr (kPolicy == kStream) __builtin_nontemporal_store(v, to_global(p));
  else *to_global(p) = v;
}

template <int C>
struct RowIO<float, C> {
  static_assert(C == 1 || C % 4 == 0, "fp32 rows move 1 or 4k elements per lane");
  template <int kPolicy = kKeep>
  static __device__ __forceinline__ void load(const float* p, float (&v)[C]) {
    if constexpr (C == 1) {
      v[0] = ld_policy<kPolicy>(p);
    } else {
#pragma unroll
      for (int q = 0; q < C / 4; ++q) {
        const f32x4 x = ld_policy<kPolicy>(reinterpret_cast<const f32x4*>(p) + q);
        v[4 * q] = x.x; v[4 * q + 1] = x.y; v[4 * q + 2] = x.z; v[4 * q + 3] = x.w;
      }
    }
  }
  template <int kPolicy = kKeep>
  static __device__ __forceinline__ void store(float* p, const float (&v)[C]) {
    if constexpr (C == 1) {
      st_policy<kPolicy>(p, v[0]);
    } else {
#pragma unroll
      for (int q = 0; q < C / 4; ++q) {
        const f32x4 x = {v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]};
        st_policy<kPolicy>(reinterpret_cast<f32x4*>(p) + q, x);
      }
    }
  }
  // The lane's 4-element pieces q at p + q * stride (stride >= 4), piece q
  // taken only when q < pieces (the rest read as zero / are not written).
  template <int kPolicy = kKeep>
  static __device__ __forceinline__ void load_pieces(const float* p, int stride, int pieces, float (&v)[C]) {
    static_assert(C % 4 == 0, "pieces of four");
#pragma unroll
    for (int q = 0; q < C / 4; ++q) {
      const f32x4 x = ld_policy<kPolicy>(reinterpret_cast<const f32x4*>(q < pieces ? p + q * stride : zero_row<float>()));
      v[4 * q] = x.x; v[4 * q + 1] = x.y; v[4 * q + 2] = x.z; v[4 * q + 3] = x.w;
    }
  }
  template <int kPolicy = kKeep>
  static __device__ __forceinline__ void store_pieces(float* p, int stride, int pieces, const float (&v)[C]) {
    static_assert(C % 4 == 0, "pieces of four");
#pragma unroll
    for (int q = 0; q < C / 4; ++q) {
      const f32x4 x = {v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]};
      if (q < pieces) st_policy<kPolicy>(reinterpret_cast<f32x4*>(p + q * stride), x);
    }
  }
};

template <int C>
struct RowIO<bf16_t, C> {
  static_assert(C == 1 || C % 8 == 0, "bf16 rows move 1 or 8k elements per lane");
  template <int kPolicy = kKeep>
  static __device__ __forceinline__ void load(const bf16_t* p, float (&v)[C]) {
    if constexpr (C == 1) {
      v[0] = bf16_to_f32(ld_policy<kPolicy>(p));
    } else {
#pragma unroll
      for (int q = 0; q < C / 8; ++q) {
        const u32x4 x = ld_policy<kPolicy>(reinterpret_cast<const u32x4*>(p) + q);
        const uint32_t w[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          v[8 * q + 2 * i] = __uint_as_float(w[i] << 16);
          v[8 * q + 2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
        }
      }
    }
  }
  template <int kPolicy = kKeep>
  static __device__ __forceinline__ void store(bf16_t* p, const float (&v)[C]) {
    if constexpr (C == 1) {
      st_policy<kPolicy>(p, f32_to_bf16(v[0]));
    } else {
#pragma unroll
      for (int q = 0; q < C / 8; ++q) {
        u32x4 w;
#pragma unroll
        for (int i = 0; i < 4; ++i)
          w[i] = (uint32_t)f32_to_bf16(v[8 * q + 2 * i]) | ((uint32_t)f32_to_bf16(v[8 * q + 2 * i + 1]) << 16);
        st_policy<kPolicy>(reinterpret_cast<u32x4*>(p) + q, w);
      }
    }
  }
};

// Compile-time tuning knobs (defaults are the ones measured best on MI355X):
// rows a lane group walks per backward chunk and per forward chunk, and the
// row elements a lane keeps in flight per iteration.
#ifndef MDL_PASSES
#define MDL_PASSES 48
#endif
#ifndef MDL_FWD_PASSES
#define MDL_FWD_PASSES 48
#endif
#ifndef MDL_ELEMS_IN_FLIGHT
#define MDL_ELEMS_IN_FLIGHT 16
#endif
// bf16 weight rows in the reduce: half as many elements (60 VGPRs, seven
// waves per SIMD instead of six): c4's apply 0.0553 -> 0.0529 ms, c3's
// unchanged; twice as many (96 VGPRs) slowed both by 10-15%.
#ifndef MDL_BF16_ELEMS_IN_FLIGHT
#define MDL_BF16_ELEMS_IN_FLIGHT 8
#endif
constexpr int kPassesPerChunk = MDL_PASSES;
constexpr int kFwdPassesPerChunk = MDL_FWD_PASSES;

// Waves per SIMD the gather/reduce kernels are compiled for: their per-wave
// work is a chain of dependent memory round trips, so throughput follows the
// number of resident waves more than the registers each one keeps.
#ifndef MDL_WAVES_PER_EU
#define MDL_WAVES_PER_EU 5
#endif
#define MDL_OCCUPANCY __attribute__((amdgpu_waves_per_eu(MDL_WAVES_PER_EU)))

// Rows per lane group per iteration for lanes of C elements.
template <int C, int kElems = MDL_ELEMS_IN_FLIGHT>
__host__ __device__ constexpr int unroll_for() {
  return C == 1 ? 4 : (kElems / C > 1 ? kElems / C : 1);
}

// ------------------------------------------------------- kernel variants --
//
// A row-access class is weight dtype x output/gradient dtype x 16-byte
// vectors or scalars.  A variant is a class x lane width: vector classes move
// C = 4 << w elements per lane (fp32 4/8/16, bf16 8/16), picked so that about
// four lanes cover a row; scalar classes move one.  A wide row then costs a
// few lanes, and the per-row bookkeeping (ids, keys, addresses, run and bag
// bounds) is paid once per 64-256 bytes instead of once per 16.  Every kernel
// that moves rows is instantiated once per variant and launched only for the
// variants present (bit `variant` of a uint32 mask).

constexpr int kWidths = 3;
#ifndef MDL_MAX_WIDTH
#define MDL_MAX_WIDTH 8
#endif
constexpr int kVariants = 6 * kWidths;

__host__ __device__ __forceinline__ int row_class(int wdtype, int odtype, bool vec) {
  const int base = wdtype == MDL_F32 ? MDL_CLASS_F32_VEC
                   : (odtype == MDL_BF16 ? MDL_CLASS_BF16_VEC : MDL_CLASS_BF16_F32_VEC);
  return base + (vec ? 0 : 1);
}

// Width index of a row of `dim` elements: C = 4 << w starts at one 16-byte
// vector of the weight type and doubles, up to MDL_MAX_WIDTH (8) elements,
// while four lanes do not cover the row and the doubled C still divides dim
// (a lane's C elements are always wholly inside the row).
__host__ __device__ __forceinline__ int width_index(int64_t dim, int wdtype, bool vec) {
  if (!vec) return 0;
  int w = wdtype == MDL_BF16 ? 1 : 0;
  while (w < kWidths - 1 && (8 << w) <= MDL_MAX_WIDTH && (int64_t)(4 << w) * 4 < dim && dim % (8 << w) == 0) ++w;
  return w;
}

__host__ __device__ __forceinline__ int variant_of(int wdtype, int odtype, bool vec, int64_t dim) {
  return row_class(wdtype, odtype, vec) * kWidths + width_index(dim, wdtype, vec);
}

// Elements per lane of a variant.
__host__ __device__ __forceinline__ int variant_elems(int v) {
  const int cls = v / kWidths;
  return (cls & 1) ? 1 : (4 << (v % kWidths));
}

template <typename TW, typename TO, int C>
struct VariantOf {
  static constexpr bool kF32 = sizeof(TW) == 4;
  static constexpr bool kOutBf16 = sizeof(TO) == 2;
  static constexpr int cls = kF32 ? (C == 1 ? MDL_CLASS_F32 : MDL_CLASS_F32_VEC)
                             : kOutBf16 ? (C == 1 ? MDL_CLASS_BF16 : MDL_CLASS_BF16_VEC)
                                        : (C == 1 ? MDL_CLASS_BF16_F32 : MDL_CLASS_BF16_F32_VEC);
  static constexpr int w = C == 1 ? 0 : (C == 4 ? 0 : (C == 8 ? 1 : 2));
  static constexpr int value = cls * kWidths + w;
};

// Kernels are launched once per row-access class present and pick the lane
// width of each chunk inside (one launch instead of one per width: separate
// launches would each pay a ramp-up and a tail).  for_each_class calls
// f.template operator()<TW, TO, kVec>() for every class with a variant bit set
// in mask (0 = all), stopping at the first non-zero return.
template <typename F>
__host__ int for_each_class(uint32_t mask, F&& f) {
  auto on = [&](int cls) { return mask == 0 || ((mask >> (cls * kWidths)) & ((1u << kWidths) - 1u)) != 0; };
  int rc = 0;
  if (!rc && on(MDL_CLASS_F32_VEC)) rc = f.template operator()<float, float, true>();
  if (!rc && on(MDL_CLASS_F32)) rc = f.template operator()<float, float, false>();
  if (!rc && on(MDL_CLASS_BF16_VEC)) rc = f.template operator()<bf16_t, bf16_t, true>();
  if (!rc && on(MDL_CLASS_BF16)) rc = f.template operator()<bf16_t, bf16_t, false>();
  if (!rc && on(MDL_CLASS_BF16_F32_VEC)) rc = f.template operator()<bf16_t, float, true>();
  if (!rc && on(MDL_CLASS_BF16_F32)) rc = f.template operator()<bf16_t, float, false>();
  return rc;
}

template <typename TW, typename TO, bool kVec>
struct ClassOf {
  static constexpr int value = VariantOf<TW, TO, kVec ? (sizeof(TW) == 4 ? 4 : 8) : 1>::cls;
};

// Calls body.template operator()<C>() with the lane width of width index w
// for a class (scalar classes: C = 1).
template <typename TW, bool kVec, typename B>
__device__ __forceinline__ void with_width(int w, B&& body) {
  if constexpr (!kVec) {
    body.template operator()<1>();
  } else {
    if constexpr (sizeof(TW) == 4 && MDL_MAX_WIDTH >= 4) {
      if (w == 0) { body.template operator()<4>(); return; }
    }
    if constexpr (MDL_MAX_WIDTH >= 8) {
      if (w == 1) { body.template operator()<8>(); return; }
    }
    if constexpr (MDL_MAX_WIDTH >= 16) {
      if (w == 2) { body.template operator()<16>(); return; }
    }
  }
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
