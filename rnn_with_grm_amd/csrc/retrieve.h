// Pieces of the retrieval kernels (retrieve.hip) shared with the window
// retrieval (retrieve_window.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "grm_hip_common.h"

namespace grmhip {

// Values per scaled float16 tile of a retrieved row: each (row, tile) has its
// own power-of-two scale.
constexpr int kScaledTile = 128;

// Exact 16-bit MFMA when both operands are exact in one 16-bit MFMA input type
// EF: the query in the arithmetic type EM must be exact in EF, and the stored
// memories split into NPART parts of EF without loss.  Otherwise fp32 MFMA.
template <class EL, class EM, class EQ>
struct MfmaPlan {
  static constexpr bool kSame = std::is_same<EL, EM>::value;
  static constexpr bool kF32 = std::is_same<EM, F32>::value;
  // EM 16-bit (then EL == EM): the query is cast to EM, EF = EM, one part.
  // EM float32: queries bf16 with fp32 / bf16 / f16 memories (3 / 1 / 2 bf16
  // parts), or f16 queries with f16 memories (one f16 part).
  static constexpr bool kBf16Q = std::is_same<EQ, BF16>::value;
  static constexpr bool kF16Both = std::is_same<EQ, F16>::value && std::is_same<EL, F16>::value;
  static constexpr bool ok = !kF32 ? kSame : (kBf16Q || kF16Both);
  using EF = typename std::conditional<!kF32, EM, typename std::conditional<kF16Both, F16, BF16>::type>::type;
  static constexpr int parts = !kF32 ? 1
                               : kF16Both ? 1
                               : std::is_same<EL, F32>::value ? 3
                               : std::is_same<EL, F16>::value ? 2
                                                              : 1;
};

// Residual + LayerNorm over scaled float16 rows:
//   out[t] = LN(h[t] + sum_r scales[t, r, c / kScaledTile] * rows[t, r, c])
// h and out in the h dtype, the LayerNorm weight and bias float32 (w NULL: no
// LayerNorm), the sum over r in order 0 .. R-1, a two-pass mean / variance in fp32.
struct FuseScaledArgs {
  const void* h;
  const uint16_t* rows;
  const float* scales;
  const void* w;
  const void* bias;
  void* out;
  int64_t n_rows;
  int routes;
  int hidden;
  int v_tiles;
  float eps;
};

int fuse_scaled(const FuseScaledArgs& a, int h_dtype, hipStream_t s);

}  // namespace grmhip
