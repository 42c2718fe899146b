// Arguments shared by the two forward scan kernels (chunk_scan.hip: value
// tiles of 16/32 columns, any dtype; chunk_scan_wide.hip: the whole 128-wide
// value tile per workgroup for 16-bit inputs).
#pragma once

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime.h>

namespace grmhip {

constexpr int CT = 64;                  // token rows per chunk tile
constexpr int PW_N = CT + 1;            // decay^0 .. decay^64
constexpr size_t kMaxLds = 160 * 1024;  // LDS per CU on gfx950

struct ChunkFwdArgs {
  const void* keys;
  const void* values;
  const void* queries;
  const void* memory;
  void* hidden;
  void* memory_out;
  float* snapshots;
  int64_t batch;
  int64_t seq_len;
  int dk;
  int dv;
  int chunk;       // tokens per chunk, 1..64
  int n_chunks;
  int snap_every;  // chunks per snapshot; 0 = no snapshots
  int n_snap;
  int v_tiles;     // workgroups per sequence
  int mem_f32;     // memory / memory_out are float32 (else the input dtype)
  int vec_m;       // memory/memory_out/snapshot rows allow 4-element vector access
  int xcd_remap;   // grid is a multiple of 8: place a sequence's tiles on one XCD
  int n_parts;     // time parts per sequence (1 = one workgroup walks the whole sequence)
  int part_chunks; // chunks per part; every part but the last is full
  float part_decay;   // decay^(part_chunks * chunk)
  float* part_states; // [batch, n_parts - 1, dv, dk]: end-state contribution of each part
  int part_starts; // part_states[q] holds M_{q+1} (combined) rather than D_q (wide kernel)
  int snap_full_lines; // value-split kernel, key_dim <= 64: snapshot stores in whole 128-byte lines (full_line_pair)
  float c;         // (1 - decay) / sqrt(d_k)
  float pw[PW_N];  // decay^n rounded from double
};

// Snapshot bytes per call from which the value-split kernel with key_dim <= 64
// stores snapshots in whole 128-byte lines: below it the writes stay in the
// 256 MB memory-side cache and the lane permutation only costs issue slots
// (config 2, value split: 48.8 -> 62.9 us); above it half-line writes cost HBM
// efficiency (64 x 8192 tokens: 290 -> 265 us, measured with key_dim 128 before
// that kernel stored its snapshots from an fp32 copy in LDS, always in whole
// lines).
constexpr int64_t kFullLineSnapBytes = 320ll << 20;

typedef float f32x4_t __attribute__((ext_vector_type(4)));

// Two 16x16 fp32 accumulator tiles of a state block, lane (g, n) holding row n,
// columns 4g .. 4g + 3 of tile x and 16 + 4g .. of tile y (so x and y are the
// two 64-byte halves of each row's 128-byte line), rearranged for two stores
// that each cover 8 rows x 128 bytes: lane (g, n) gets 16-byte chunk
// 2g + (n >> 3) of row n & 7 (oa) and of row 8 + (n & 7) (ob).  A DPP row
// rotate by 8 moves rows n +- 8 within each 16-lane row; the 32- and 16-lane
// swaps then gather the chunks across the four lane groups.
__device__ __forceinline__ void full_line_pair(f32x4_t x, f32x4_t y, int n, f32x4_t& oa, f32x4_t& ob) {
  constexpr int kRowRor8 = 0x128;
  const bool half = (n >> 3) != 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float xr = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x[i]), kRowRor8, 0xf, 0xf, false));
    const float yr = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(y[i]), kRowRor8, 0xf, 0xf, false));
    const auto a32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(half ? xr : x[i]),
                                                      __float_as_uint(half ? yr : y[i]), false, false);
    const auto a16 = __builtin_amdgcn_permlane16_swap(a32[0], a32[1], false, false);
    oa[i] = __uint_as_float(half ? a16[1] : a16[0]);
    const auto b32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(half ? x[i] : xr),
                                                      __float_as_uint(half ? y[i] : yr), false, false);
    const auto b16 = __builtin_amdgcn_permlane16_swap(b32[0], b32[1], false, false);
    ob[i] = __uint_as_float(half ? b16[1] : b16[0]);
  }
}

// Value columns per workgroup of the wide kernel.
constexpr int kWideDv = 128;

// The wide kernel covers 16-bit inputs with key_dim <= 128 and 16-byte
// aligned rows (key_dim and value_dim multiples of 8).
bool wide_supported(int in_dtype, int64_t key_dim, int64_t value_dim, bool vec);

// Launches the wide kernel: with a.n_parts > 1 the state pass (and, for many
// parts, the combine step), then the full pass.
int launch_scan_wide(const ChunkFwdArgs& a, int in_dtype, int mem_dtype, hipStream_t stream);

// Value columns per workgroup of the value-split kernel, and the chunks its
// loads run ahead of the chunk being scanned.
constexpr int kVsplitDv = 32;
constexpr int kVsplitPrefetch = 4;

// The value-split kernel covers what the wide kernel covers with value_dim a
// multiple of kVsplitDv; one workgroup walks each (sequence, value tile).
bool vsplit_supported(int in_dtype, int64_t key_dim, int64_t value_dim, bool vec);

// Launches the value-split kernel (a.n_parts must be 1, a.v_tiles = value_dim / kVsplitDv).
int launch_scan_vsplit(const ChunkFwdArgs& a, int in_dtype, hipStream_t stream);

}  // namespace grmhip
