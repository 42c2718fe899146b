// Shared device-side helpers for the GRM hot-path kernels (gfx950 / CDNA4).
//
// Element traits, 8-element operand fragments for the 16x16 MFMA family, and
// the error/launch bookkeeping used by every C-ABI entry point.
//
// Fragment convention (used by every MFMA kernel in this library):
//   * a "fragment" covers a 16-row tile and a 32-wide slice of the reduction
//     axis; lane l = 16*g + n holds row n and 8 reduction slots s = 0..7.
//   * which logical reduction index a (g, s) slot stands for is a per-GEMM
//     permutation; the A and B operands of one GEMM always use the same one,
//     so the sum is unchanged.
//   * the 16x16 accumulator (f32x4) has lane (g, n), register r holding
//     D[4g + r][n].  Read as a fragment it is row n, reduction index 4g + r,
//     which is what lets an MFMA output feed the next MFMA without an LDS
//     round trip.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace grmhip {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

// Element tags.  The numeric values match the dtype enum of grm_hip.h.
struct F32 { static constexpr int code = 0; };
struct F16 { static constexpr int code = 1; };
struct BF16 { static constexpr int code = 2; };

template <class E> struct ET;

template <> struct ET<F32> {
  using raw = float;
  __device__ __forceinline__ static float to_f(raw x) { return x; }
  __device__ __forceinline__ static raw from_f(float f) { return f; }
};

template <> struct ET<F16> {
  using raw = uint16_t;
  __device__ __forceinline__ static float to_f(raw x) {
    return static_cast<float>(__builtin_bit_cast(_Float16, x));
  }
  __device__ __forceinline__ static raw from_f(float f) {
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
  }
};

template <> struct ET<BF16> {
  using raw = uint16_t;
  __device__ __forceinline__ static float to_f(raw x) {
    return __uint_as_float(static_cast<uint32_t>(x) << 16);
  }
  // Round to nearest even, the rounding torch uses for float -> bfloat16.
  __device__ __forceinline__ static raw from_f(float f) {
    return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
  }
};

// Two values in a 16-bit input dtype packed into 32 bits (first in the low
// half): one conversion instruction for the pair, rounding as from_f.
template <class E>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
  static_assert(sizeof(typename ET<E>::raw) == 2, "16-bit types");
  typedef float f32x2_t __attribute__((ext_vector_type(2)));
  const f32x2_t v = {a, b};
  if constexpr (std::is_same_v<E, BF16>) {
    typedef __bf16 h2_t __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, h2_t));
  } else {
    typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, h2_t));
  }
}

// Eight consecutive elements of one row (16 B for 16-bit types, 32 B for f32).
template <class E> struct U8 {
  typename ET<E>::raw e[8];
};

// Eight MFMA reduction slots of one lane.
template <class E> struct Frag8 {
  typename ET<E>::raw e[8];
};

template <class E>
__device__ __forceinline__ void zero_u8(U8<E>& u) {
#pragma unroll
  for (int i = 0; i < 8; ++i) u.e[i] = 0;
}

// Load 8 elements row[col .. col+8) with zero fill past `ncols` or when the
// row is out of range.  `vec` says the caller has checked 16 B alignment of
// every row start and that ncols is a multiple of 8.
template <class E>
__device__ __forceinline__ U8<E> load_u8(const typename ET<E>::raw* row, int col, int ncols,
                                         bool row_ok, bool vec) {
  U8<E> u;
  if (row_ok && vec && col + 8 <= ncols) {
    if constexpr (sizeof(typename ET<E>::raw) == 2) {
      uint4 v = *reinterpret_cast<const uint4*>(row + col);
      u = __builtin_bit_cast(U8<E>, v);
    } else {
      const float4* p = reinterpret_cast<const float4*>(row + col);
      float4 a = p[0];
      float4 b = p[1];
      u.e[0] = a.x; u.e[1] = a.y; u.e[2] = a.z; u.e[3] = a.w;
      u.e[4] = b.x; u.e[5] = b.y; u.e[6] = b.z; u.e[7] = b.w;
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      u.e[i] = (row_ok && col + i < ncols) ? row[col + i] : static_cast<typename ET<E>::raw>(0);
    }
  }
  return u;
}

// 16x16 MFMA over one 8-slot fragment pair: acc += A * B^T (rows of A are the
// output's row index m, rows of B its column index n).
__device__ __forceinline__ f32x4 mfma8(const Frag8<BF16>& a, const Frag8<BF16>& b, f32x4 acc) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), acc, 0, 0, 0);
}

__device__ __forceinline__ f32x4 mfma8(const Frag8<F16>& a, const Frag8<F16>& b, f32x4 acc) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                __builtin_bit_cast(f16x8, b), acc, 0, 0, 0);
}

// fp32 inputs: eight 16x16x4 MFMAs, slot s of every lane forming the s-th one.
__device__ __forceinline__ f32x4 mfma8(const Frag8<F32>& a, const Frag8<F32>& b, f32x4 acc) {
#pragma unroll
  for (int s = 0; s < 8; ++s) {
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.e[s], b.e[s], acc, 0, 0, 0);
  }
  return acc;
}

// Two 4-element LDS runs (8 B each for 16-bit types) into one fragment:
// slots 0..3 from p0, slots 4..7 from p1.
template <class E>
__device__ __forceinline__ Frag8<E> lds_frag_4x2(const typename ET<E>::raw* p0,
                                                 const typename ET<E>::raw* p1) {
  if constexpr (sizeof(typename ET<E>::raw) == 2) {
    const uint2 lo = *reinterpret_cast<const uint2*>(p0);
    const uint2 hi = *reinterpret_cast<const uint2*>(p1);
    return __builtin_bit_cast(Frag8<E>, make_uint4(lo.x, lo.y, hi.x, hi.y));
  } else {
    const float4 lo = *reinterpret_cast<const float4*>(p0);
    const float4 hi = *reinterpret_cast<const float4*>(p1);
    Frag8<E> f;
    f.e[0] = lo.x; f.e[1] = lo.y; f.e[2] = lo.z; f.e[3] = lo.w;
    f.e[4] = hi.x; f.e[5] = hi.y; f.e[6] = hi.z; f.e[7] = hi.w;
    return f;
  }
}

// Four consecutive elements converted from fp32 and stored with one access.
template <class E>
__device__ __forceinline__ void store4_raw(typename ET<E>::raw* p, f32x4 v) {
  if constexpr (sizeof(typename ET<E>::raw) == 2) {
    uint2 q;
    q.x = pack2<E>(v[0], v[1]);
    q.y = pack2<E>(v[2], v[3]);
    *reinterpret_cast<uint2*>(p) = q;
  } else {
    *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
  }
}

// ---------------------------------------------------------------------------
// Raw buffer access (gfx9 family).  A resource covers [base, base + bytes);
// loads outside it return zero and stores outside it are dropped, so row and
// column masks become offset selects instead of branches.
constexpr int kBufOOB = 0x7ffffff0;  // an offset past every resource used here

// 64-bit integer min / max for device code.  HIP's min<int64_t> / max<int64_t>
// (an explicit template argument) compile to double arithmetic on the vector
// unit, and a buffer resource built from such a result is treated as
// divergent: every load through it gets a readfirstlane loop.
__host__ __device__ __forceinline__ int64_t min_i64(int64_t a, int64_t b) { return a < b ? a : b; }
__host__ __device__ __forceinline__ int64_t max_i64(int64_t a, int64_t b) { return a > b ? a : b; }

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0),
                                           static_cast<int>(bytes), 0x00020000);
}

// Rows dealt `per` lanes each (per a power of two, at most 64) to a workgroup
// whose first row is `block_first`: this lane's row, its wavefront's first row
// (wave-uniform) and how many of the wavefront's rows lie below n_rows.  A
// buffer resource built per lane from tid / per is divergent as far as the
// compiler can tell, and every load through it gets a readfirstlane loop; one
// built at the wavefront's first row and spanning its rows (wave_rows_rsrc) is
// uniform, and each lane adds local * row_bytes to its offsets.  Rows past
// n_rows fall outside it: they read zeros and their stores drop.
struct WaveRows {
  int64_t row;    // this lane's row
  int64_t first;  // the wavefront's first row
  int local;      // row - first
  int count;      // rows of the wavefront below n_rows, 0 .. 64 / per
};

__device__ __forceinline__ WaveRows wave_rows(int64_t block_first, int per, int64_t n_rows) {
  WaveRows w;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
  const int rows_per_wave = 64 / per;
  w.local = static_cast<int>(threadIdx.x & 63) / per;
  w.first = block_first + static_cast<int64_t>(wave) * rows_per_wave;
  w.row = w.first + w.local;
  const int64_t left = n_rows - w.first;
  w.count = static_cast<int>(left < 0 ? 0 : (left < rows_per_wave ? left : rows_per_wave));
  return w;
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t wave_rows_rsrc(const void* base, const WaveRows& w,
                                                                 uint32_t row_bytes) {
  return make_rsrc(static_cast<const char*>(base) + w.first * row_bytes, static_cast<uint32_t>(w.count) * row_bytes);
}

// Eight consecutive elements starting at byte offset `off` (OOB -> zeros).
template <class E>
__device__ __forceinline__ U8<E> buf_load8(__amdgpu_buffer_rsrc_t r, int off) {
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  if constexpr (sizeof(typename ET<E>::raw) == 2) {
    const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
    return __builtin_bit_cast(U8<E>, v);
  } else {
    const u32x4 a = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
    const u32x4 b = __builtin_amdgcn_raw_buffer_load_b128(r, off + 16, 0, 0);
    U8<E> u;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      u.e[i] = __uint_as_float(a[i]);
      u.e[4 + i] = __uint_as_float(b[i]);
    }
    return u;
  }
}

// One element at byte offset `off` (OOB -> zero).
template <class E>
__device__ __forceinline__ typename ET<E>::raw buf_load1(__amdgpu_buffer_rsrc_t r, int off) {
  if constexpr (sizeof(typename ET<E>::raw) == 2) {
    return __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0);
  } else {
    return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
  }
}

// Four consecutive elements converted from fp32 (OOB -> dropped).
template <class E>
__device__ __forceinline__ void buf_store4(__amdgpu_buffer_rsrc_t r, int off, f32x4 v) {
  if constexpr (sizeof(typename ET<E>::raw) == 2) {
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    u32x2 q;
    q[0] = pack2<E>(v[0], v[1]);
    q[1] = pack2<E>(v[2], v[3]);
    __builtin_amdgcn_raw_buffer_store_b64(q, r, off, 0, 0);
  } else {
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    u32x4 q;
#pragma unroll
    for (int i = 0; i < 4; ++i) q[i] = __float_as_uint(v[i]);
    __builtin_amdgcn_raw_buffer_store_b128(q, r, off, 0, 0);
  }
}

template <class E>
__device__ __forceinline__ void buf_store1(__amdgpu_buffer_rsrc_t r, int off, float v) {
  if constexpr (sizeof(typename ET<E>::raw) == 2) {
    __builtin_amdgcn_raw_buffer_store_b16(ET<E>::from_f(v), r, off, 0, 0);
  } else {
    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), r, off, 0, 0);
  }
}

__device__ __forceinline__ int lane_id() { return static_cast<int>(threadIdx.x) & 63; }

}  // namespace grmhip

// ---------------------------------------------------------------------------
// Host-side bookkeeping shared by the entry points (defined in grm_capi.hip).
namespace grmhip {
void set_error(const char* fmt, ...);
void count_launch();
int check_launch(const char* what);
}  // namespace grmhip
