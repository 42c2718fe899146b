// Segment-window retrieval, gfx950: retrieve_fuse for indices that come from
// segment routing over a small archive window, without one row per (query, route).
//
//   out[b, t, :] = LN(h_online[b, t, :] + sum_r gates[b, t, r] * M[b, idx[b, t, r]] q[b, t])
//
// the reference's retriever followed by its aggregator in residual mode
// (grm/core/paper_grm.py:229,301-313,604-611; grm/core/aggregator.py:67-145), for
// the routing of its segment loop (paper_grm.py:702-728 -> _route_chunk, :566-589):
// query t sees the archive entries [lo(t), hi(t)), hi(t) = base + t / segment_len,
// lo(t) = max(0, hi(t) - capacity).
//
// retrieve_fuse sorts (query, route) pairs by archive entry, applies each entry
// to the queries that selected it and writes one float16 row per pair, which a
// second pass sums per query: at config 4 that is 268 MB written and read back
// per layer.  Here the 96 queries of a block see at most capacity + 95 /
// segment_len + 1 entries, so one workgroup per (block, 128-value tile) walks
// those entries in index order and adds each entry's products into float32
// accumulators in LDS (one row per query).  Wave w owns value rows [16 w, 16 w +
// 16) of the tile: for entry j the queries that selected j (a list built in LDS)
// are the columns of 16x16x32 MFMAs whose A operand is the entry's 16 rows, read
// from a copy of the windows' entries laid out in the MFMA's fragment order (one
// pass before; the fragment order of the row-major entry would need 64-byte half
// lines, at half the load rate).  The products are exact 16-bit products (float32
// entries split into three bf16 parts; float16 entries with bf16 queries take
// float16 MFMA with each query scaled by a power of two), float32 accumulation.
// Each query appears at most once per entry and each wave only touches its own
// rows, so the per-query sums run in entry order with no atomics: the result
// does not depend on the order of the lists.  The tile's sums then leave as
// float16 scaled by a power of two per (query, tile), retrieve_fuse's row
// format, and the same residual + LayerNorm pass (fuse_scaled, one route)
// finishes the rows.
#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <type_traits>

#include "grm_hip.h"
#include "grm_hip_common.h"
#include "retrieve.h"

namespace grmhip {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int WR_THREADS = 512;       // 8 waves, 16 value rows each
constexpr int WR_TOK = 96;            // queries per workgroup (two workgroups' LDS fit one CU)
constexpr int WR_V = kScaledTile;     // value rows per workgroup
constexpr int WR_AS = WR_V + 4;       // accumulator row stride (floats)
constexpr int WR_SPAN_MAX = 256;      // archive entries one block's windows may span
constexpr int WR_ROUTES_MAX = 32;
constexpr int kDeadItem = 1 << 30;    // a padding work item: no pairs
static_assert(WR_V == 16 * (WR_THREADS / 64), "one 16-row slice per wave");
static_assert(WR_TOK % 16 == 0, "the output pass takes 16 queries per wave round");

struct WinArgs {
  const void* msw;      // the window's entries in fragment order: [batch, n_ent, ent_units, 16 bytes]
  const int64_t* idx;   // [batch, n_query, routes]
  const void* q;        // [batch, n_query, dk]
  const float* gates;   // [batch, n_query, routes]
  uint16_t* rows;       // [batch * n_query, dv] float16, scaled per (row, tile)
  float* scales;        // [batch * n_query, v_tiles]
  int32_t* bad;
  int64_t segments;
  int64_t n_query;
  int64_t seg_len;
  int64_t base;
  int64_t capacity;
  int routes;
  int dv;
  int dk;
  int v_tiles;
  int n_blocks;  // query blocks per sequence
  int64_t ent_lo;  // first entry of the copy
  int n_ent;
  int ent_units;   // 16-byte units per copied entry
};

// Operand plan per (memories, queries) dtype pair: the MFMA input type EF, the
// parts the memories split into (one unless float32), and whether the queries
// enter as float16 scaled by a power of two per query (float16 memories with
// bf16 queries: the memories then need no split, and a bf16 query component
// is exact in float16 once scaled, unless it is below 2^-29 of the query's
// largest magnitude, where float16 keeps it to 2^-40 of that magnitude).
template <class EL, class EQ>
struct WinPlan {
  static constexpr bool qscale = std::is_same_v<EL, F16> && std::is_same_v<EQ, BF16>;
  static constexpr bool ok = qscale || MfmaPlan<EL, F32, EQ>::ok;
  using EF = typename std::conditional<qscale, F16, typename MfmaPlan<EL, F32, EQ>::EF>::type;
  static constexpr int parts = qscale ? 1 : MfmaPlan<EL, F32, EQ>::parts;
};

template <int DKP>
struct WinLds {
  static constexpr int QS = DKP + 8;  // query row stride (16-bit elements)
  static constexpr int acc_bytes = WR_TOK * WR_AS * 4;
  static constexpr int q_bytes = WR_TOK * QS * 2;
  // work items, padded with dead ones to a multiple of four plus four read ahead
  __host__ __device__ static int items_max(int routes) { return WR_SPAN_MAX + (WR_TOK * routes + 15) / 16 + 8; }
  static int bytes(int routes) {
    const int pairs = WR_TOK * routes;
    // query scales, codes, list tokens (int16, padded), gates, scales, offsets, work items, counters
    return acc_bytes + q_bytes + WR_TOK * 4 + pairs * 4 + (pairs * 2 + 15) / 16 * 16 + pairs * 4 +
           pairs * 4 + (WR_SPAN_MAX + 1) * 4 + items_max(routes) * 4 + 16;
  }
};

template <class EL, class EQ, int DKP>
__global__ __launch_bounds__(WR_THREADS) void retrieve_window_kernel(const WinArgs a) {
  using Plan = WinPlan<EL, EQ>;
  using EF = typename Plan::EF;
  constexpr int NPART = Plan::parts;
  constexpr bool QSCALE = Plan::qscale;
  using rawl = typename ET<EL>::raw;
  using rawq = typename ET<EQ>::raw;
  using L = WinLds<DKP>;
  constexpr int QS = L::QS;
  constexpr int NSTEP = DKP / 32;                 // 32-key MFMA steps
  constexpr int UPS = sizeof(rawl) == 2 ? 1 : 2;  // 16-byte loads per lane per step
  static_assert(sizeof(rawq) == 2, "16-bit queries");
  extern __shared__ __align__(16) unsigned char lds[];
  const int R = a.routes;
  const int pairs_max = WR_TOK * R;
  float* acc = reinterpret_cast<float*>(lds);
  uint16_t* qs = reinterpret_cast<uint16_t*>(lds + L::acc_bytes);
  float* tscale = reinterpret_cast<float*>(lds + L::acc_bytes + L::q_bytes);
  int32_t* code = reinterpret_cast<int32_t*>(tscale + WR_TOK);
  int16_t* ltok = reinterpret_cast<int16_t*>(code + pairs_max);
  float* lgate = reinterpret_cast<float*>(reinterpret_cast<unsigned char*>(ltok) + (pairs_max * 2 + 15) / 16 * 16);
  float* lsc = lgate + pairs_max;
  int* off = reinterpret_cast<int*>(lsc + pairs_max);
  int* items = off + WR_SPAN_MAX + 1;
  int* counters = items + L::items_max(R);  // [0] bad pairs, [1] work items

  const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, n = lane & 15;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  // Workgroup order: consecutive logical ids (the blocks of one sequence and one value
  // tile) on one XCD, so that the workgroups resident on an XCD at a time read one
  // tile of one sequence's entries, which its L2 then holds.
  const int lin = blockIdx.x, total = gridDim.x;
  const int logical = (total % 8 == 0) ? (lin % 8) * (total / 8) + lin / 8 : lin;
  const int per_b = a.n_blocks * a.v_tiles;
  const int64_t b = logical / per_b;
  const int vt = (logical % per_b) / a.n_blocks, blk = logical % a.n_blocks;
  const int64_t t0 = static_cast<int64_t>(blk) * WR_TOK;
  const int nt = static_cast<int>(min_i64(WR_TOK, a.n_query - t0));
  const int64_t hi_b = a.base + (t0 + nt - 1) / a.seg_len;
  const int64_t lo_b = max_i64(0, a.base + t0 / a.seg_len - a.capacity);
  const int span = static_cast<int>(hi_b - lo_b);  // <= WR_SPAN_MAX (host check)
  const int dk = a.dk, dv = a.dv;

  // ---- every global input of the block first (queries, indices, gates), then the
  // accumulators and the histogram zeroed while they arrive; the queries into LDS
  constexpr int UPR = DKP / 8;                         // 16-byte units per query row; UPR lanes share a row
  constexpr int QPT = (WR_TOK * UPR + WR_THREADS - 1) / WR_THREADS;  // query units per thread
  constexpr int PPT = (WR_TOK * WR_ROUTES_MAX + WR_THREADS - 1) / WR_THREADS;  // pairs per thread at most
  const int n_pairs = nt * R;
  u32x4 qv[QPT];
  int64_t jv[PPT];
  float gv[PPT];
  {
    const rawq* qb = static_cast<const rawq*>(a.q) + (b * a.n_query + t0) * dk;
    const __amdgpu_buffer_rsrc_t rq = make_rsrc(qb, static_cast<uint32_t>(nt * dk * 2));
#pragma unroll
    for (int i = 0; i < QPT; ++i) {
      const int e = tid + WR_THREADS * i, t = e / UPR, u = e % UPR;
      qv[i] = __builtin_amdgcn_raw_buffer_load_b128(rq, (t < nt && 8 * u < dk) ? (t * dk + 8 * u) * 2 : kBufOOB, 0, 0);
    }
    const int64_t pbase = (b * a.n_query + t0) * R;
#pragma unroll
    for (int i = 0; i < PPT; ++i) {
      const int e = tid + WR_THREADS * i;
      jv[i] = e < n_pairs ? a.idx[pbase + e] : -1;
      gv[i] = e < n_pairs ? a.gates[pbase + e] : 0.f;
    }
  }
  for (int e = tid; e < WR_TOK * WR_AS / 4; e += WR_THREADS)
    reinterpret_cast<f32x4*>(acc)[e] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int e = tid; e <= WR_SPAN_MAX; e += WR_THREADS) off[e] = 0;
  if (tid < 2) counters[tid] = 0;
  {
#pragma unroll
    for (int i = 0; i < QPT; ++i) {
      const int e = tid + WR_THREADS * i, t = e / UPR, u = e % UPR;
      const u32x4 v = qv[i];
      if constexpr (QSCALE) {
        // q * 2^sh as float16, the largest magnitude of the row in [2^14, 2^15)
        float x[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          x[2 * i] = ET<BF16>::to_f(static_cast<uint16_t>(v[i] & 0xffffu));
          x[2 * i + 1] = ET<BF16>::to_f(static_cast<uint16_t>(v[i] >> 16));
        }
        float m = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) m = fmaxf(m, fabsf(x[i]));
#pragma unroll
        for (int o = 1; o < UPR; o <<= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
        int ex = 0;
        (void)frexpf(m, &ex);
        const int sh = min(max(15 - ex, -100), 100);
        const u32x4 h = u32x4{pack2<F16>(ldexpf(x[0], sh), ldexpf(x[1], sh)), pack2<F16>(ldexpf(x[2], sh), ldexpf(x[3], sh)),
                              pack2<F16>(ldexpf(x[4], sh), ldexpf(x[5], sh)), pack2<F16>(ldexpf(x[6], sh), ldexpf(x[7], sh))};
        if (t < WR_TOK) {
          *reinterpret_cast<u32x4*>(qs + t * QS + 8 * u) = h;
          if (u == 0) tscale[t] = ldexpf(1.f, -sh);
        }
      } else {
        if (t < WR_TOK) *reinterpret_cast<u32x4*>(qs + t * QS + 8 * u) = v;
      }
    }
  }
  __syncthreads();

  // ---- the block's pairs: an index outside its query's window is bad (-2), a
  // negative one an empty slot (-1), otherwise its entry relative to lo_b; then a pair
  // repeating an earlier route of its query is bad too, and every good pair takes a
  // slot in its entry's bin.
  int* relv = reinterpret_cast<int*>(lsc);  // the pairs' entries, before the list's scales are written
#pragma unroll
  for (int i = 0; i < PPT; ++i) {
    const int e = tid + WR_THREADS * i;
    if (e < n_pairs) {
      const int64_t t = t0 + e / R, j = jv[i];
      const int64_t hi = a.base + t / a.seg_len, lo = max_i64(0, hi - a.capacity);
      relv[e] = j < 0 ? -1 : (j >= lo && j < hi) ? static_cast<int>(j - lo_b) : -2;
    }
  }
  __syncthreads();
  {
    int bad = 0;
    for (int e = tid; e < n_pairs; e += WR_THREADS) {
      const int rel = relv[e];
      int c = -1;
      if (rel >= 0) {
        const int r = e % R, first = e - r;
        bool ok = true;
        for (int r2 = 0; r2 < r; ++r2) ok = ok && relv[first + r2] != rel;
        if (ok) {
          c = (rel << 16) | atomicAdd(&off[rel], 1);
        } else {
          ++bad;
        }
      } else if (rel == -2) {
        ++bad;
      }
      code[e] = c;
    }
    if (bad) atomicAdd(&counters[0], bad);
  }
  __syncthreads();
  // Exclusive scan of the bins (wave 0, four bins per lane), off[span] = pairs; then the
  // work items: one per 16 pairs of an entry, (entry, first pair, pairs - 1) packed.
  if (tid < 64) {
    int v[4], nti[4], sum = 0, tiles = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int bin = 4 * tid + i;
      v[i] = bin < span ? off[bin] : 0;
      nti[i] = (v[i] + 15) / 16;
      sum += v[i];
      tiles += nti[i];
    }
    int incl = sum, tincl = tiles;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int y = __shfl_up(incl, d, 64), ty = __shfl_up(tincl, d, 64);
      if (tid >= d) {
        incl += y;
        tincl += ty;
      }
    }
    int run = incl - sum, item = tincl - tiles;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int bin = 4 * tid + i;
      if (bin < span) off[bin] = run;
      for (int u = 0; u < nti[i]; ++u)
        items[item++] = (bin << 17) | ((run + 16 * u) << 4) | (min(16, v[i] - 16 * u) - 1);
      run += v[i];
    }
    if (tid == 63) {
      off[span] = incl;
      counters[1] = tincl;
#pragma unroll
      for (int i = 0; i < 8; ++i) items[tincl + i] = kDeadItem;
    }
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < PPT; ++i) {
    const int e = tid + WR_THREADS * i;
    const int c = e < n_pairs ? code[e] : -1;
    if (c >= 0) {
      const int pos = off[c >> 16] + (c & 0xffff);
      const int t = e / R;
      ltok[pos] = static_cast<int16_t>(t);
      lgate[pos] = gv[i];
      if constexpr (QSCALE) lsc[pos] = tscale[t];
    }
  }
  if (vt == 0 && tid == 0 && a.bad != nullptr && counters[0] > 0) atomicAdd(a.bad, counters[0]);
  __syncthreads();

  // ---- the work items in entry order, each wave on its own 16 value rows, in a
  // pipeline with the same instructions every step (items past the end are dead:
  // their loads read nothing, their sums are not stored), so that every wait is
  // for exactly the data it needs.  Step k: item k's accumulator row is read, item
  // k + 4's word, k + 3's entry rows (global) and list slots, k + 1's query
  // fragments, then item k's products and update.
  const int n_items = __builtin_amdgcn_readfirstlane(counters[1]);
  const int n_steps = (n_items + 3) / 4 * 4;
  struct Slot {
    int word;  // (entry, first pair, pairs - 1) or kDeadItem
    u32x4 a[NSTEP * UPS];
    int tok;
    float gate, sc;
    bool live;
    Frag8<EF> q[NSTEP];
  };
  // The entry copy holds lane (g, n)'s 16 bytes of step s (and half u of a float32
  // step) at unit ((row block * NSTEP + s) * UPS + u) * 64 + 16 g + n: every load is
  // 1 KB of whole lines.
  const unsigned char* swb = static_cast<const unsigned char*>(a.msw) + b * a.n_ent * static_cast<int64_t>(a.ent_units) * 16;
  const int rblk = vt * (WR_V / 16) + w;  // this wave's 16-row block
  auto load_rows = [&](Slot& sl) {
    const int word = __builtin_amdgcn_readfirstlane(sl.word);
    const bool dead = word == kDeadItem;
    const int64_t e = dead ? 0 : lo_b + (word >> 17) - a.ent_lo;
    const __amdgpu_buffer_rsrc_t rm = make_rsrc(swb + e * a.ent_units * 16, static_cast<uint32_t>(a.ent_units * 16));
#pragma unroll
    for (int s = 0; s < NSTEP; ++s)
#pragma unroll
      for (int u = 0; u < UPS; ++u)
        sl.a[s * UPS + u] = __builtin_amdgcn_raw_buffer_load_b128(
            rm, dead ? kBufOOB : (((rblk * NSTEP + s) * UPS + u) * 64 + lane) * 16, 0, 0);
  };
  auto load_meta = [&](Slot& sl) {
    const int word = __builtin_amdgcn_readfirstlane(sl.word);
    sl.live = word != kDeadItem && n <= (word & 15);
    const int p = sl.live ? ((word >> 4) & 0x1fff) + n : 0;
    sl.tok = sl.live ? ltok[p] : 0;
    sl.gate = lgate[p];
    if constexpr (QSCALE) sl.sc = lsc[p];
  };
  auto load_q = [&](Slot& sl) {
#pragma unroll
    for (int s = 0; s < NSTEP; ++s)
      sl.q[s] = __builtin_bit_cast(Frag8<EF>, *reinterpret_cast<const u32x4*>(qs + sl.tok * QS + 32 * s + 8 * g));
  };
  auto products = [&](const Slot& sl) {
    f32x4 d = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < NSTEP; ++s) {
      if constexpr (NPART == 1 && UPS == 1) {
        d = mfma8(__builtin_bit_cast(Frag8<EF>, sl.a[s]), sl.q[s], d);
      } else {
        // float32 rows: NPART exact parts of the MFMA input type
        float x[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          x[i] = __uint_as_float(sl.a[2 * s][i]);
          x[4 + i] = __uint_as_float(sl.a[2 * s + 1][i]);
        }
        Frag8<EF> af[NPART];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          float rest = x[e];
#pragma unroll
          for (int part = 0; part < NPART; ++part) {
            const typename ET<EF>::raw h = ET<EF>::from_f(rest);
            af[part].e[e] = h;
            rest -= ET<EF>::to_f(h);
          }
        }
#pragma unroll
        for (int part = 0; part < NPART; ++part) d = mfma8(af[part], sl.q[s], d);
      }
    }
    return d;  // d[r]: value row 16 w + 4 g + r of query tok
  };
  // cur = item k (rows, slots and query fragments in), n1 = item k + 1 (rows loading,
  // slots in), n2 = item k + 2 (rows loading, slots in), n3 = item k + 3 (word in)
  auto step = [&](int k, Slot& cur, Slot& n1, Slot& n2, Slot& n3) {
    f32x4* ap = reinterpret_cast<f32x4*>(acc + cur.tok * WR_AS + 16 * w + 4 * g);
    f32x4 o = *ap;  // after the previous item's store (one wave's LDS operations stay in order)
    const int w4 = items[k + 4];
    load_rows(n3);
    load_meta(n3);
    load_q(n1);
    const f32x4 d = products(cur);
#pragma unroll
    for (int r = 0; r < 4; ++r) o[r] = fmaf(cur.gate, QSCALE ? d[r] * cur.sc : d[r], o[r]);
    if (cur.live) *ap = o;
    cur.word = w4;
  };
  Slot s0, s1, s2, s3;
  s0.word = items[0];
  s1.word = items[1];
  s2.word = items[2];
  s3.word = items[3];
  load_rows(s0);
  load_meta(s0);
  load_rows(s1);
  load_meta(s1);
  load_rows(s2);
  load_meta(s2);
  load_q(s0);
  for (int k = 0; k < n_steps; k += 4) {
    step(k, s0, s1, s2, s3);
    step(k + 1, s1, s2, s3, s0);
    step(k + 2, s2, s3, s0, s1);
    step(k + 3, s3, s0, s1, s2);
  }
  __syncthreads();

  // ---- the tile's sums out as float16 rows scaled so that each (query, tile)'s
  // largest magnitude lies in [2^14, 2^15), with the inverse power of two beside
  // them: 32 lanes per query, four values each.
  const int half = lane >> 5, hl = lane & 31;
  const int vcols = min(WR_V, dv - vt * WR_V);
  constexpr int OPW = WR_TOK / (2 * (WR_THREADS / 64));  // queries per half-wave
  f32x4 val[OPW];
  float m[OPW];
#pragma unroll
  for (int i = 0; i < OPW; ++i) {
    val[i] = *reinterpret_cast<const f32x4*>(acc + (2 * w + half + 16 * i) * WR_AS + 4 * hl);
    m[i] = fmaxf(fmaxf(fabsf(val[i][0]), fabsf(val[i][1])), fmaxf(fabsf(val[i][2]), fabsf(val[i][3])));
  }
#pragma unroll
  for (int o = 1; o < 32; o <<= 1) {
    float t[OPW];
#pragma unroll
    for (int i = 0; i < OPW; ++i) t[i] = __shfl_xor(m[i], o, 64);
#pragma unroll
    for (int i = 0; i < OPW; ++i) m[i] = fmaxf(m[i], t[i]);
  }
#pragma unroll
  for (int i = 0; i < OPW; ++i) {
    const int t = 2 * w + half + 16 * i;
    if (t >= nt) continue;
    int ex = 0;
    (void)frexpf(m[i], &ex);
    const int sh = min(max(15 - ex, -100), 100);
    const int64_t row = b * a.n_query + t0 + t;
    uint16_t* dst = a.rows + row * dv + vt * WR_V + 4 * hl;
    if (4 * hl + 4 <= vcols) {
      uint2 qv;
      qv.x = pack2<F16>(ldexpf(val[i][0], sh), ldexpf(val[i][1], sh));
      qv.y = pack2<F16>(ldexpf(val[i][2], sh), ldexpf(val[i][3], sh));
      *reinterpret_cast<uint2*>(dst) = qv;
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (4 * hl + r < vcols) dst[r] = ET<F16>::from_f(ldexpf(val[i][r], sh));
    }
    if (hl == 0) a.scales[row * a.v_tiles + vt] = ldexpf(1.f, -sh);
  }
}

// The window's entries [ent_lo, ent_lo + n_ent) of every sequence in the fragment
// order of retrieve_window_kernel's loads (zero rows past dv, zero keys past dk).
template <class EL, int DKP>
__global__ __launch_bounds__(256) void window_copy_kernel(const void* mem, void* msw, int64_t segments,
                                                          int64_t ent_lo, int n_ent, int dv, int dk, int units) {
  using rawl = typename ET<EL>::raw;
  constexpr int NSTEP = DKP / 32;
  constexpr int UPS = sizeof(rawl) == 2 ? 1 : 2;
  const int64_t b = blockIdx.z, e = blockIdx.y;
  const __amdgpu_buffer_rsrc_t rs =
      make_rsrc(static_cast<const rawl*>(mem) + (b * segments + ent_lo + e) * dv * dk,
                static_cast<uint32_t>(dv * dk * sizeof(rawl)));
  u32x4* dst = static_cast<u32x4*>(msw) + (b * n_ent + e) * units;
  for (int u = blockIdx.x * 256 + threadIdx.x; u < units; u += gridDim.x * 256) {
    const int lane = u & 63, rest = u >> 6;
    const int uu = rest % UPS, s = (rest / UPS) % NSTEP, rb = rest / (UPS * NSTEP);
    const int row = 16 * rb + (lane & 15), k = 32 * s + 8 * (lane >> 4) + 4 * uu;
    const int off = (row < dv && k < dk) ? (row * dk + k) * static_cast<int>(sizeof(rawl)) : kBufOOB;
    dst[u] = __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0);
  }
}

template <class EL, int DKP>
int launch_window_copy(const void* mem, const WinArgs& a, int64_t batch, hipStream_t s) {
  if (a.n_ent == 0) return GRM_HIP_OK;
  const dim3 grid(static_cast<unsigned>((a.ent_units + 255) / 256), static_cast<unsigned>(a.n_ent),
                  static_cast<unsigned>(batch));
  hipLaunchKernelGGL((window_copy_kernel<EL, DKP>), grid, dim3(256), 0, s, mem, const_cast<void*>(a.msw), a.segments,
                     a.ent_lo, a.n_ent, a.dv, a.dk, a.ent_units);
  return check_launch("segment_retrieve_fuse(entry copy)");
}

template <class EL, class EQ, int DKP>
int launch_window(const void* mem, const WinArgs& a, int64_t batch, hipStream_t s) {
  if constexpr (!WinPlan<EL, EQ>::ok) {
    set_error("segment_retrieve_fuse: needs bf16 queries (or f16 queries with f16 memories)");
    return GRM_HIP_EUNSUPPORTED;
  } else {
    auto kern = &retrieve_window_kernel<EL, EQ, DKP>;
    const int lds = WinLds<DKP>::bytes(a.routes);
    if (lds > 160 * 1024) {
      set_error("segment_retrieve_fuse: %d routes need %d bytes of LDS", a.routes, lds);
      return GRM_HIP_EUNSUPPORTED;
    }
    static bool attr_set = false;
    if (!attr_set) {
      hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                         hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
      if (e != hipSuccess) {
        set_error("segment_retrieve_fuse: hipFuncSetAttribute failed: %s", hipGetErrorString(e));
        return static_cast<int>(e);
      }
      attr_set = true;
    }
    const int rc = launch_window_copy<EL, DKP>(mem, a, batch, s);
    if (rc != GRM_HIP_OK) return rc;
    const int64_t grid = batch * a.n_blocks * a.v_tiles;
    hipLaunchKernelGGL(kern, dim3(static_cast<unsigned>(grid)), dim3(WR_THREADS), lds, s, a);
    return check_launch("segment_retrieve_fuse(window sums)");
  }
}

template <class EL, class EQ>
int dispatch_window_dk(const void* mem, const WinArgs& a, int64_t batch, hipStream_t s) {
  if (a.dk <= 32) return launch_window<EL, EQ, 32>(mem, a, batch, s);
  if (a.dk <= 64) return launch_window<EL, EQ, 64>(mem, a, batch, s);
  return launch_window<EL, EQ, 128>(mem, a, batch, s);
}

template <class EL>
int dispatch_window_q(const void* mem, const WinArgs& a, int64_t batch, int q_dtype, hipStream_t s) {
  switch (q_dtype) {
    case GRM_HIP_F16: return dispatch_window_dk<EL, F16>(mem, a, batch, s);
    case GRM_HIP_BF16: return dispatch_window_dk<EL, BF16>(mem, a, batch, s);
    default:
      set_error("segment_retrieve_fuse: needs 16-bit queries");
      return GRM_HIP_EUNSUPPORTED;
  }
}

int64_t align16w(int64_t n) { return (n + 15) / 16 * 16; }

// The entries any query of the call can see: [max(0, base - capacity), base + (n_query - 1) / segment_len).
void window_entries(int64_t n_query, int64_t segment_len, int64_t base, int64_t capacity, int64_t* lo, int64_t* n) {
  *lo = std::max<int64_t>(0, base - capacity);
  *n = n_query > 0 ? std::max<int64_t>(0, base + (n_query - 1) / segment_len - *lo) : 0;
}

// 16-byte units of one entry's copy: 16-row blocks of the padded value width, the
// padded key width's steps, two halves per float32 step.
int64_t copy_units(int64_t value_dim, int64_t key_dim, int mem_dtype) {
  const int64_t dkp = key_dim <= 32 ? 32 : key_dim <= 64 ? 64 : 128;
  const int64_t v_tiles = (value_dim + kScaledTile - 1) / kScaledTile;
  return v_tiles * (kScaledTile / 16) * (dkp / 32) * (mem_dtype == GRM_HIP_F32 ? 2 : 1) * 64;
}

}  // namespace
}  // namespace grmhip

using namespace grmhip;

extern "C" int64_t grm_hip_segment_retrieve_fuse_workspace(int64_t batch, int64_t n_query, int64_t value_dim,
                                                           int64_t key_dim, int64_t segment_len, int64_t base,
                                                           int64_t capacity, int mem_dtype) {
  if (batch <= 0 || n_query <= 0 || value_dim <= 0 || key_dim < 1 || segment_len < 1 || base < 0 || capacity < 1)
    return 0;
  const int64_t tiles = (value_dim + kScaledTile - 1) / kScaledTile;
  int64_t lo, n_ent;
  window_entries(n_query, segment_len, base, capacity, &lo, &n_ent);
  return align16w(batch * n_query * value_dim * 2) + align16w(batch * n_query * tiles * 4) +
         batch * n_ent * copy_units(value_dim, key_dim, mem_dtype) * 16;
}

extern "C" int grm_hip_segment_retrieve_fuse(const void* memories, const int64_t* indices, const void* queries,
                                             const float* gates, const void* h_online, const void* ln_weight,
                                             const void* ln_bias, void* out, void* workspace, int64_t workspace_bytes,
                                             int64_t batch, int64_t segments, int64_t n_query, int64_t routes,
                                             int64_t value_dim, int64_t key_dim, int64_t segment_len, int64_t base,
                                             int64_t capacity, int mem_dtype, int q_dtype, int h_dtype, float eps,
                                             int32_t* bad_index_count, void* stream) {
  if (batch < 0 || segments < 0 || n_query < 0 || routes < 0 || value_dim < 0 || key_dim < 1) {
    set_error("segment_retrieve_fuse: negative size or key_dim < 1");
    return GRM_HIP_EINVAL;
  }
  if (segment_len < 1 || base < 0 || capacity < 1) {
    set_error("segment_retrieve_fuse: needs segment_len >= 1, base >= 0 and capacity >= 1");
    return GRM_HIP_EINVAL;
  }
  if (mem_dtype < GRM_HIP_F32 || mem_dtype > GRM_HIP_BF16 || q_dtype < GRM_HIP_F32 || q_dtype > GRM_HIP_BF16 ||
      h_dtype < GRM_HIP_F32 || h_dtype > GRM_HIP_BF16) {
    set_error("segment_retrieve_fuse: unsupported dtypes mem=%d q=%d h=%d", mem_dtype, q_dtype, h_dtype);
    return GRM_HIP_EUNSUPPORTED;
  }
  if (n_query > 0 && base + (n_query - 1) / segment_len > segments) {
    set_error("segment_retrieve_fuse: windows past the archive (base + (n_query - 1) / segment_len > segments)");
    return GRM_HIP_EINVAL;
  }
  const int64_t span_bound = std::min(capacity, base + (n_query > 0 ? (n_query - 1) / segment_len : 0)) +
                             (WR_TOK - 1) / segment_len + 1;
  if (key_dim > 128 || key_dim % 8 != 0 || value_dim % 8 != 0 || value_dim > 2048 || routes > WR_ROUTES_MAX ||
      span_bound > WR_SPAN_MAX) {
    set_error("segment_retrieve_fuse: needs key_dim <= 128 and a multiple of 8, value_dim a multiple of 8 and <= "
              "2048, routes <= %d and capacity + 127 / segment_len + 1 <= %d (use retrieve_fuse)",
              WR_ROUTES_MAX, WR_SPAN_MAX);
    return GRM_HIP_EUNSUPPORTED;
  }
  const int64_t rows = batch * n_query;
  if (rows == 0 || value_dim == 0) return GRM_HIP_OK;
  if (h_online == nullptr || out == nullptr || (routes > 0 && (indices == nullptr || gates == nullptr)) ||
      queries == nullptr || (segments > 0 && memories == nullptr)) {
    set_error("segment_retrieve_fuse: null pointer");
    return GRM_HIP_EINVAL;
  }
  const int64_t v_tiles = (value_dim + kScaledTile - 1) / kScaledTile;
  const int64_t n_blocks = (n_query + WR_TOK - 1) / WR_TOK;
  if (batch * n_blocks * v_tiles > INT32_MAX || n_query * key_dim * 2 > INT32_MAX ||
      value_dim * key_dim * 4 > INT32_MAX) {
    set_error("segment_retrieve_fuse: sizes exceed one launch");
    return GRM_HIP_EINVAL;
  }
  const int64_t need = grm_hip_segment_retrieve_fuse_workspace(batch, n_query, value_dim, key_dim, segment_len, base,
                                                               capacity, mem_dtype);
  if (workspace == nullptr || workspace_bytes < need || reinterpret_cast<uintptr_t>(workspace) % 16 != 0) {
    set_error("segment_retrieve_fuse: workspace of %lld bytes (16-byte aligned) required", (long long)need);
    return GRM_HIP_EINVAL;
  }
  const int hb = h_dtype == GRM_HIP_F32 ? 4 : 2;
  if (reinterpret_cast<uintptr_t>(h_online) % 16 != 0 || reinterpret_cast<uintptr_t>(out) % 16 != 0 ||
      reinterpret_cast<uintptr_t>(queries) % 16 != 0 || reinterpret_cast<uintptr_t>(memories) % 16 != 0 ||
      (ln_weight != nullptr && reinterpret_cast<uintptr_t>(ln_weight) % 16 != 0) ||
      (ln_bias != nullptr && reinterpret_cast<uintptr_t>(ln_bias) % 16 != 0) || (value_dim * hb) % 16 != 0) {
    set_error("segment_retrieve_fuse: memories, queries, h_online, out and the LayerNorm parameters must be 16-byte "
              "aligned");
    return GRM_HIP_EUNSUPPORTED;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  uint16_t* rows16 = static_cast<uint16_t*>(workspace);
  float* scales = reinterpret_cast<float*>(static_cast<unsigned char*>(workspace) + align16w(rows * value_dim * 2));
  int64_t ent_lo, n_ent;
  window_entries(n_query, segment_len, base, capacity, &ent_lo, &n_ent);
  const int64_t units = copy_units(value_dim, key_dim, mem_dtype);
  if (units * 16 > INT32_MAX || n_ent > 65535 || batch > 65535) {
    set_error("segment_retrieve_fuse: sizes exceed one launch");
    return GRM_HIP_EINVAL;
  }
  WinArgs a;
  memset(&a, 0, sizeof(a));
  a.msw = static_cast<unsigned char*>(workspace) + align16w(rows * value_dim * 2) + align16w(rows * v_tiles * 4);
  a.ent_lo = ent_lo;
  a.n_ent = static_cast<int>(n_ent);
  a.ent_units = static_cast<int>(units);
  a.idx = indices;
  a.q = queries;
  a.gates = gates;
  a.rows = rows16;
  a.scales = scales;
  a.bad = bad_index_count;
  a.segments = segments;
  a.n_query = n_query;
  a.seg_len = segment_len;
  a.base = base;
  a.capacity = capacity;
  a.routes = static_cast<int>(routes);
  a.dv = static_cast<int>(value_dim);
  a.dk = static_cast<int>(key_dim);
  a.v_tiles = static_cast<int>(v_tiles);
  a.n_blocks = static_cast<int>(n_blocks);
  int rc;
  switch (mem_dtype) {
    case GRM_HIP_F32: rc = dispatch_window_q<F32>(memories, a, batch, q_dtype, s); break;
    case GRM_HIP_F16: rc = dispatch_window_q<F16>(memories, a, batch, q_dtype, s); break;
    default: rc = dispatch_window_q<BF16>(memories, a, batch, q_dtype, s); break;
  }
  if (rc != GRM_HIP_OK) return rc;
  FuseScaledArgs f;
  f.h = h_online;
  f.rows = rows16;
  f.scales = scales;
  f.w = ln_weight;
  f.bias = ln_bias;
  f.out = out;
  f.n_rows = rows;
  f.routes = 1;
  f.hidden = static_cast<int>(value_dim);
  f.v_tiles = static_cast<int>(v_tiles);
  f.eps = eps;
  return fuse_scaled(f, h_dtype, s);
}
