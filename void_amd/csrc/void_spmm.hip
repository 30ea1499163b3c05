// void_spmm.hip — gfx950 block-sparse SpMM kernels (INT8 and FP8 E4M3) and
// the C ABI declared in include/void_amd.h.
//
// One workgroup = 4 wave64s = one work item (a block-row, or a chunk of a
// long block-row) x one 128-column panel of C.  The waves take the item's
// 32x32 tiles round-robin; each tile is one 32x32x32 int8 MFMA (or two
// 32x32x16 fp8 MFMAs) per 32 output columns, four MFMAs per wave per tile.
//
// B operand without LDS: a lane owning MFMA column j and k-group g loads 16
// consecutive rows k = 32*kb + 16*g + t of four adjacent columns
// (4j .. 4j+3) as 16 dwords, then transposes the 4x4 byte blocks in
// registers (v_perm_b32) into four k-contiguous 16-byte operands, one per
// column.  MFMA c (c = 0..3) therefore produces output columns 4j + c, and in
// the epilogue every lane owns four adjacent columns, so C is written with
// full 16-byte stores.  A operand: lane (j, g) reads bytes [16g, 16g+16) of
// tile row j, the same k set, so the k permutation agrees for A and B.
// A column-major B (activations stored token-major) is loaded as 16 bytes
// per column directly, with no transpose.
//
// Latency: the work item (128 bytes) carries the block columns of its first
// 24 tiles, so the B addresses of the first batches come with the item; the
// epilogue's scale, bias and row-mean factors are loaded before the tile
// loop; each wave keeps the loads of kBatch tiles in flight.
//
// Cross-wave reduction goes through LDS (4 x 16 KB).  Rows that the planner
// split into several items write partial tiles to a workspace with
// agent-coherent stores; the last chunk to arrive (agent-scope atomic
// counter) sums the partials in chunk order and applies the epilogue, so
// results do not depend on timing.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <type_traits>
#include <vector>

#include "void_amd.h"
#include "lds_dma.h"

extern "C" size_t void_workspace_bytes(int32_t n_split_tiles, int32_t n_slots, int32_t N);

namespace {

constexpr int kTile = 32;
constexpr int kWaves = 4;
constexpr int kColsPerLane = 4;
constexpr int kPanel = 32 * kColsPerLane;  // 128 output columns per workgroup
constexpr int kThreads = 64 * kWaves;
constexpr int kBatch = 5;                  // tiles whose loads one wave keeps in flight
constexpr int kInline = VOID_ITEM_INLINE_COLS;
constexpr int kRowsPerWave = kTile / kWaves;  // epilogue rows per wave

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v2i __attribute__((ext_vector_type(2)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v2f __attribute__((ext_vector_type(2)));

// Tile element types: int8 and E4M3 tiles times a B of the same type; fp32
// tiles times fp32 B (float SpMM); E4M3 tiles times fp32 B (kEltFp8F32, the
// reference's FP8 SpMM with a float B); bf16 or fp16 tiles times a B of the
// same type (float SpMM on 16-bit tensors, on the 16-bit MFMA); E4M3 tiles
// times a bf16 or fp16 B (the reference's FP8 SpMM with a 16-bit B, on the
// 16-bit MFMA with A decoded exactly).
enum Elt { kEltI8 = 0, kEltFp8 = 1, kEltF32 = 2, kEltFp8F32 = 3, kEltBf16 = 4, kEltF16 = 5, kEltFp8Bf16 = 6,
           kEltFp8F16 = 7 };

struct Params {
  const uint8_t* tiles;
  const float* a_scale;
  const int32_t* row_ptr;
  const int32_t* col_idx;
  const uint8_t* b;
  const float* b_scale_vec;
  const float* bias;
  void* c;
  const void_work_item* items;
  unsigned* counters;
  void* partials;
  unsigned long long* trace;  // per-workgroup phase timestamps (instrumented builds only)
  int64_t ldb;
  int64_t ldc;
  float b_scale;
  int32_t per_tensor_a;
  int32_t M, N, K;
  int32_t n_panels;
  int32_t activation;
  int32_t n_items;
  int32_t panel_group;  // panels one XCD's share of the grid covers (see wg_tile)
  int32_t item_piles;   // XCDs among which one panel group's items are dealt (see wg_map)
  int32_t xcd_exact;    // grid laid out per XCD (see wg_map)
  int32_t bias_per_row;  // float kernel: bias indexed by output row
  int32_t pair_snake;    // exact layout: second half of an XCD's share reversed (see wg_map)
};

#ifdef VOID_TRACE
// Realtime stamps are kept in scalar registers and written once at exit, so
// that nothing is stored before the kernel's loads (a store would stop the
// compiler from using scalar loads for the read-only inputs).
#define TRACE_DECL unsigned long long tr0 = 0, tr1 = 0, tr2 = 0, tr3 = 0, tr4 = 0, tr5 = 0, tr6 = 0, tr7 = 0
#ifdef VOID_TRACE_CLK
// Clock probe: point 0 also reads the shader clock counter (s_memtime) into
// slot 1, point 4 into slot 2, so that (t2 - t1) / (t4 - t0) is the engine
// clock over a workgroup's life; points 1 and 2 record nothing.
#define TRACE_POINT(k)                                                                              \
  do {                                                                                              \
    if ((k) == 0) asm volatile("s_memrealtime %0\n\ts_memtime %1\n\ts_waitcnt lgkmcnt(0)" : "=s"(tr0), "=s"(tr1)); \
    else if ((k) == 4) asm volatile("s_memrealtime %0\n\ts_memtime %1\n\ts_waitcnt lgkmcnt(0)" : "=s"(tr4), "=s"(tr2)); \
    else if ((k) != 1 && (k) != 2) asm volatile("s_memrealtime %0\n\ts_waitcnt lgkmcnt(0)" : "=s"(tr##k));        \
  } while (0)
#else
#define TRACE_POINT(k) asm volatile("s_memrealtime %0\n\ts_waitcnt lgkmcnt(0)" : "=s"(tr##k))
#endif
#define TRACE_TAG(v)                                                           \
  do {                                                                         \
    unsigned x_, h_;                                                           \
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(x_));          \
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_HW_ID)" : "=s"(h_));           \
    tr7 = (unsigned long long)(v) | ((unsigned long long)(x_ & 15) << 8) |     \
          ((unsigned long long)h_ << 40);                                      \
  } while (0)
#define TRACE_FLUSH()                                                              \
  do {                                                                             \
    if (p.trace && threadIdx.x == 0) {                                             \
      unsigned long long* t_ = p.trace + (size_t)blockIdx.x * 8;                   \
      t_[0] = tr0; t_[1] = tr1; t_[2] = tr2; t_[3] = tr3;                          \
      t_[4] = tr4; t_[5] = tr5; t_[6] = tr6; t_[7] = tr7;                \
    }                                                                              \
  } while (0)
#else
#define TRACE_DECL \
  do {             \
  } while (0)
#define TRACE_POINT(k) \
  do {                 \
  } while (0)
#define TRACE_TAG(v) \
  do {               \
  } while (0)
#define TRACE_FLUSH() \
  do {                \
  } while (0)
#endif

// Workgroups are dispatched round-robin over the 8 XCDs, each with its own
// L2.  xcd_remap turns the hardware id into a logical id such that every XCD
// runs one contiguous range of logical ids.
__device__ __forceinline__ int xcd_remap(int h, int G) {
  const int per = G >> 3, rem = G & 7;
  const int x = h & 7, s = h >> 3;
  return x < rem ? x * (per + 1) + s : rem * (per + 1) + (x - rem) * per + s;
}

// Position r of the work list dealt round-robin into `piles` piles laid end
// to end -> index into the longest-first list.  Pile p holds list entries
// p, p + piles, p + 2 piles, ...; the first n % piles piles have one entry
// more than the rest.
__device__ __forceinline__ int undeal(int r, int n, int piles) {
  if (piles <= 1) return r;
  const int q = n / piles, rem = n - q * piles;
  const int big = rem * (q + 1);  // entries in the longer piles
  int pile, k;
  if (r < big) {
    pile = r / (q + 1);
    k = r - pile * (q + 1);
  } else {  // q >= 1 here: r < n = big + (piles - rem) q
    const int r2 = r - big;
    pile = rem + r2 / q;
    k = r2 - (pile - rem) * q;
  }
  return k * piles + pile;
}

// Logical id -> (work item, panel).  Panels are taken in groups of
// panel_group (about n_panels / 8, so that one XCD's range covers one group);
// within a group the order is item-major.  An XCD then reads the B columns
// of its group's panels only (they stay in its L2), and the panels of one
// item run back to back on the same XCD, sharing the item's A tiles.
// item_piles > 1 (the XCDs that share one group): the group's items are
// dealt so that each of those XCDs runs a balanced, still longest-first
// share of the list rather than a contiguous slice of it.
__device__ __forceinline__ void wg_tile(int L, int n_items, int n_panels, int pgrp, int item_piles, int& item,
                                        int& panel) {
  const int full = n_panels / pgrp;  // groups of exactly pgrp panels
  const int gsize = n_items * pgrp;
  int g = L / gsize;
  int w = pgrp;
  int r = L - g * gsize;
  if (g >= full) {  // trailing group of n_panels % pgrp panels
    g = full;
    w = n_panels - full * pgrp;
    r = L - full * gsize;
  }
  const int pos = r / w;
  panel = g * pgrp + (r - pos * w);
  item = undeal(pos, n_items, item_piles);
}

// Hardware workgroup id -> (work item, panel); false for the padding
// workgroups of the exact layout below, which do nothing.
//
// Exact layout (xcd_exact, set when rows were split and the panel groups
// divide the 8 XCDs evenly): XCD x = h % 8 serves group x / item_piles and
// runs every item_piles-th item of the longest-first list, starting at item
// x % item_piles, one whole item (its panel_group panels back to back) after
// another.  The grid is 8 x (that share's workgroups, rounded up), so every
// XCD's share is a longest-first slice of equal length.  Unsplit grids of
// one resident round (pair_snake) take the same layout with the second half
// of each XCD's share reversed: the dispatcher gives each CU of an XCD one
// workgroup of the first half and then one of the second (read from
// HW_REG_HW_ID in an instrumented build: workgroups s and s + 32 of an XCD's
// 64 share a CU), so a CU's pair is a long and a short row.  Against
// contiguous ranges, where one XCD of a panel took all its longest rows, c2
// went 8.6-8.8 -> 7.9-8.1 us and c3 10.9-11.1 -> 10.2-10.7 us cold.
// Otherwise each XCD runs a contiguous range of logical ids (xcd_remap),
// mapped by wg_tile.
__device__ __forceinline__ bool wg_map(const Params& p, int& item, int& panel) {
  const int h = (int)blockIdx.x;
  if (p.xcd_exact) {
    const int x = h & 7, s = h >> 3;
    const int piles = p.item_piles, pg = p.panel_group;
    int k = s / pg;
    panel = (x / piles) * pg + (s - k * pg);
    if (p.pair_snake) {
      const int share = (p.n_items + piles - 1) / piles, half = (share + 1) >> 1;
      k = k < half ? k : share - 1 - (k - half);
    }
    item = k * piles + x % piles;
    return item < p.n_items;
  }
  wg_tile(xcd_remap(h, (int)gridDim.x), p.n_items, p.n_panels, p.panel_group, p.item_piles, item, panel);
  return true;
}

// wg_map on the layout fields packed into three scalar kernel arguments
// (map_word: xcd_exact | pair_snake << 1 | item_piles << 2 | panel_group << 8),
// which the column-group kernel takes ahead of Params so that they can be
// preloaded into SGPRs with the work list's address: its first work-item read
// then waits for no kernel-argument load.
__device__ __forceinline__ bool wg_map_args(int map_word, int n_items, int n_panels, int& item, int& panel) {
  const int h = (int)blockIdx.x;
  const int piles = (map_word >> 2) & 63, pg = map_word >> 8;
  if (map_word & 1) {
    const int x = h & 7, s = h >> 3;
    int k = s / pg;
    panel = (x / piles) * pg + (s - k * pg);
    if (map_word & 2) {
      const int share = (n_items + piles - 1) / piles, half = (share + 1) >> 1;
      k = k < half ? k : share - 1 - (k - half);
    }
    item = k * piles + x % piles;
    return item < n_items;
  }
  wg_tile(xcd_remap(h, (int)gridDim.x), n_items, n_panels, pg, piles, item, panel);
  return true;
}

// Split-row fix-up ordering (all three kernels).  The protocol uses no
// release/acquire fences (at agent scope on gfx950 they write back and
// invalidate the XCD's whole L2); it is ordered by completion instead:
//  1. every partial-block access carries agent scope (sc1, the encoding of a
//     relaxed agent-scope atomic), so each location is coherent across the
//     8 XCDs;
//  2. publish_wait: vmcnt(0) returns only when this wave's partial stores
//     are acknowledged at that scope; the barrier that follows puts every
//     wave's acknowledgement before thread 0 issues the arrival counter's
//     RMW;
//  3. the last arriver issues its partial loads only after the RMW has
//     returned (its result decides, through LDS and a barrier, whether the
//     loads run at all), and the hardware issues a wave's memory operations
//     in order and does not speculate loads, so they observe every
//     acknowledged store.
// The hardware waits alone leave the compiler free to move relaxed accesses
// to other addresses across them; the "memory" clobbers below forbid that.
__device__ __forceinline__ void publish_wait() {
  asm volatile("s_waitcnt vmcnt(0) expcnt(0) lgkmcnt(0)" ::: "memory");
}
__device__ __forceinline__ void compiler_order() { asm volatile("" ::: "memory"); }

// 4x4 byte transpose: r_i holds bytes (B[k+i][n+0..3]); c_n gets (B[k+0..3][n]).
__device__ __forceinline__ void transpose4x4(uint32_t r0, uint32_t r1, uint32_t r2, uint32_t r3,
                                             uint32_t& c0, uint32_t& c1, uint32_t& c2,
                                             uint32_t& c3) {
  // v_perm_b32(s0, s1, sel): byte selector 0..3 picks from s1, 4..7 from s0.
  const uint32_t lo01 = __builtin_amdgcn_perm(r1, r0, 0x05010400u);  // r0.0 r1.0 r0.1 r1.1
  const uint32_t hi01 = __builtin_amdgcn_perm(r1, r0, 0x07030602u);  // r0.2 r1.2 r0.3 r1.3
  const uint32_t lo23 = __builtin_amdgcn_perm(r3, r2, 0x05010400u);
  const uint32_t hi23 = __builtin_amdgcn_perm(r3, r2, 0x07030602u);
  c0 = __builtin_amdgcn_perm(lo23, lo01, 0x05040100u);
  c1 = __builtin_amdgcn_perm(lo23, lo01, 0x07060302u);
  c2 = __builtin_amdgcn_perm(hi23, hi01, 0x05040100u);
  c3 = __builtin_amdgcn_perm(hi23, hi01, 0x07060302u);
}

// Raw operand registers of one tile for one lane, as loaded from memory.
// Row-major B: r[i] holds B[k0+i][col0 .. col0+3] (one dword per row);
// column-major B: r[4c+q] holds B[k0+4q .. k0+4q+3][col0+c].
struct Raw {
  v4i a;
  uint32_t r[16];
  int krow;  // rows r[0 .. krow) lie inside K
};

// Issue the loads of tile t (block column kb) without consuming them.
// Columns at or beyond N read a clamped valid address: they only feed MFMA
// output columns that are never stored.  Rows at or beyond K read a clamped
// valid row; they meet the zero padding of the A tile, and the fp8 path
// zeroes them explicitly (a NaN code times zero is still NaN).
template <bool BCOL, bool VEC>
__device__ __forceinline__ void load_raw(const Params& p, int t, int kb, int j, int g, int col0, Raw& f) {
  f.a = *reinterpret_cast<const v4i*>(p.tiles + (size_t)t * (kTile * kTile) + j * kTile + g * 16);
  const int k0 = kb * kTile + g * 16;
  const bool kfull = kb * kTile + kTile <= p.K;  // uniform: the whole 32-row slab of B exists
  f.krow = 16;
  if constexpr (!BCOL) {
    if constexpr (VEC) {
      const uint8_t* base = p.b + (col0 < p.N ? col0 : 0);
      if (kfull) {
        const uint8_t* bp = base + (int64_t)k0 * p.ldb;
#pragma unroll
        for (int i = 0; i < 16; ++i) f.r[i] = *reinterpret_cast<const uint32_t*>(bp + i * p.ldb);
      } else {
        f.krow = p.K - k0;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int kk = k0 + i;
          const int kc = kk < p.K ? kk : p.K - 1;
          f.r[i] = *reinterpret_cast<const uint32_t*>(base + (int64_t)kc * p.ldb);
        }
      }
    } else {
      const uint8_t* bp = p.b + (int64_t)k0 * p.ldb + col0;
      const int krem = p.K - k0;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        uint32_t w = 0;
#pragma unroll
        for (int c = 0; c < 4; ++c)
          if (i < krem && col0 + c < p.N) w |= (uint32_t)bp[i * p.ldb + c] << (8 * c);
        f.r[i] = w;
      }
    }
  } else {
#pragma unroll
    for (int c = 0; c < kColsPerLane; ++c) {
      if constexpr (VEC) {
        // Host guarantees K % 32 == 0, ldb % 16 == 0 and a 16-byte aligned b.
        const int cc = col0 + c < p.N ? col0 + c : 0;
        const v4i v = *reinterpret_cast<const v4i*>(p.b + (int64_t)cc * p.ldb + k0);
#pragma unroll
        for (int q = 0; q < 4; ++q) f.r[4 * c + q] = (uint32_t)v[q];
      } else {
        const uint8_t* bp = p.b + (int64_t)(col0 + c) * p.ldb + k0;
        const int krem = p.K - k0;
        uint32_t w[4] = {0, 0, 0, 0};
#pragma unroll
        for (int i = 0; i < 16; ++i)
          if (i < krem && col0 + c < p.N) w[i >> 2] |= (uint32_t)bp[i] << (8 * (i & 3));
#pragma unroll
        for (int q = 0; q < 4; ++q) f.r[4 * c + q] = w[q];
      }
    }
  }
}

// MFMA operands of one tile: b[c] = 16 k-contiguous bytes of column col0 + c.
struct Frag {
  v4i a;
  v4i b[kColsPerLane];
};

template <int ELT, bool BCOL>
__device__ __forceinline__ void to_frag(const Raw& raw, Frag& f) {
  f.a = raw.a;
  if constexpr (!BCOL) {
    uint32_t r[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) r[i] = (ELT == kEltFp8 && i >= raw.krow) ? 0u : raw.r[i];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      uint32_t c0, c1, c2, c3;
      transpose4x4(r[4 * q], r[4 * q + 1], r[4 * q + 2], r[4 * q + 3], c0, c1, c2, c3);
      f.b[0][q] = (int)c0;
      f.b[1][q] = (int)c1;
      f.b[2][q] = (int)c2;
      f.b[3][q] = (int)c3;
    }
  } else {
#pragma unroll
    for (int c = 0; c < kColsPerLane; ++c)
#pragma unroll
      for (int q = 0; q < 4; ++q) f.b[c][q] = (int)raw.r[4 * c + q];
  }
}

__device__ __forceinline__ long pack2(int lo, int hi) {
  return (long)(((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo);
}

// acc[c] += tile product for output columns col0 + c.
template <int ELT, int EPI>
struct Accum;

template <int EPI>
struct Accum<kEltI8, EPI> {
  static constexpr bool kInt = (EPI != VOID_EPI_PER_BLOCK);
  using Reg = typename std::conditional<kInt, v16i, v16f>::type;
  __device__ __forceinline__ static void step(Reg (&acc)[kColsPerLane], const Frag& f, float s) {
#pragma unroll
    for (int c = 0; c < kColsPerLane; ++c) {
      if constexpr (kInt) {
        acc[c] = __builtin_amdgcn_mfma_i32_32x32x32_i8(f.a, f.b[c], acc[c], 0, 0, 0);
      } else {
        const v16i z = {};
        const v16i part = __builtin_amdgcn_mfma_i32_32x32x32_i8(f.a, f.b[c], z, 0, 0, 0);
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[c][r] = __builtin_fmaf(s, (float)part[r], acc[c][r]);
      }
    }
  }
};

template <int EPI>
struct Accum<kEltFp8, EPI> {
  static constexpr bool kInt = false;
  using Reg = v16f;
  __device__ __forceinline__ static void step(Reg (&acc)[kColsPerLane], const Frag& f, float s) {
    const long a0 = pack2(f.a[0], f.a[1]), a1 = pack2(f.a[2], f.a[3]);
#pragma unroll
    for (int c = 0; c < kColsPerLane; ++c) {
      const v16f z = {};
      v16f part = __builtin_amdgcn_mfma_f32_32x32x16_fp8_fp8(a0, pack2(f.b[c][0], f.b[c][1]), z, 0, 0, 0);
      part = __builtin_amdgcn_mfma_f32_32x32x16_fp8_fp8(a1, pack2(f.b[c][2], f.b[c][3]), part, 0, 0, 0);
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[c][r] = __builtin_fmaf(s, part[r], acc[c][r]);
    }
  }
};

// sigmoid(t) = 1 / (1 + e^-t) = 1 / (1 + 2^(-t log2 e)) on the hardware
// exp2 and reciprocal (1 ulp each).  Rounding -t log2 e costs |t| 2^-24 ln 2
// relative error at most, where sigmoid is e^t-small; elsewhere it is
// damped.  Saturates to exactly 1 and 0; NaN propagates.
__device__ __forceinline__ float sigmoid_fast(float t) {
  return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(t * -1.4426950408889634f));
}

// fusion.py:38-43: inner = 0.7978845608 (x + 0.044715 x^3) and
// 0.5 x (1 + tanh(inner)), with tanh(u) = 2 sigmoid(2u) - 1, which is
// x sigmoid(2 inner) = x / (1 + 2^t), t = x (c0 + c1 x^2),
// c0 = -2 0.7978845608 log2(e), c1 = 0.044715 c0: three VALU operations
// and two transcendentals.
__device__ __forceinline__ float gelu_fast(float x) {
  constexpr float c0 = -2.0f * 0.7978845608f * 1.4426950408889634f;
  constexpr float c1 = 0.044715f * c0;
  const float t = x * __builtin_fmaf(x * x, c1, c0);
  return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(t));
}

__device__ __forceinline__ float activate(float x, int act) {
  if (act == VOID_ACT_RELU) return fmaxf(x, 0.0f);
  if (act == VOID_ACT_GELU) return gelu_fast(x);
  if (act == VOID_ACT_SILU) return x * sigmoid_fast(x);
  return x;
}

// The activation of n values, with the (wave-uniform) choice made once, so
// the element loop has no branches.
template <int N>
__device__ __forceinline__ void activate_all(float (&x)[N], int act) {
  if (act == VOID_ACT_RELU) {
#pragma unroll
    for (int r = 0; r < N; ++r) x[r] = fmaxf(x[r], 0.0f);
  } else if (act == VOID_ACT_GELU) {
#pragma unroll
    for (int r = 0; r < N; ++r) x[r] = gelu_fast(x[r]);
  } else if (act == VOID_ACT_SILU) {
#pragma unroll
    for (int r = 0; r < N; ++r) x[r] = x[r] * sigmoid_fast(x[r]);
  }
}

// gfx950's v_cvt_pk_bf16_f32: round to nearest even, NaN stays a (quiet) NaN.
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float x) {
  const __bf16 h = (__bf16)x;
  uint16_t u;
  __builtin_memcpy(&u, &h, 2);
  return u;
}

__device__ __forceinline__ uint32_t f32_to_f16_bits(float x) {
  _Float16 h = (_Float16)x;
  uint16_t u;
  __builtin_memcpy(&u, &h, 2);
  return u;
}

template <int OUT, bool VEC>
__device__ __forceinline__ void store4(const Params& p, int grow, int col, const float (&v)[4],
                                       const int (&vi)[4]) {
  if (grow >= p.M) return;
  if constexpr (VEC) {
    if (col >= p.N) return;
    if constexpr (OUT == VOID_DT_F32) {
      *reinterpret_cast<v4f*>(static_cast<float*>(p.c) + (int64_t)grow * p.ldc + col) =
          v4f{v[0], v[1], v[2], v[3]};
    } else if constexpr (OUT == VOID_DT_I32) {
      *reinterpret_cast<v4i*>(static_cast<int*>(p.c) + (int64_t)grow * p.ldc + col) =
          v4i{vi[0], vi[1], vi[2], vi[3]};
    } else {
      uint32_t h[4];
#pragma unroll
      for (int c = 0; c < 4; ++c)
        h[c] = OUT == VOID_DT_BF16 ? f32_to_bf16_bits(v[c]) : f32_to_f16_bits(v[c]);
      uint2 w;
      w.x = h[0] | (h[1] << 16);
      w.y = h[2] | (h[3] << 16);
      *reinterpret_cast<uint2*>(static_cast<uint16_t*>(p.c) + (int64_t)grow * p.ldc + col) = w;
    }
  } else {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      if (col + c >= p.N) break;
      const int64_t off = (int64_t)grow * p.ldc + col + c;
      if constexpr (OUT == VOID_DT_F32) static_cast<float*>(p.c)[off] = v[c];
      else if constexpr (OUT == VOID_DT_I32) static_cast<int*>(p.c)[off] = vi[c];
      else if constexpr (OUT == VOID_DT_BF16) static_cast<uint16_t*>(p.c)[off] = (uint16_t)f32_to_bf16_bits(v[c]);
      else static_cast<uint16_t*>(p.c)[off] = (uint16_t)f32_to_f16_bits(v[c]);
    }
  }
}

// ---- B through LDS (row-major B, N and ldb multiples of 16) --------------
// A tile's 32 x 128 B slab is read with four 16-byte loads per lane (lane l,
// load q: row 8q + l/8, bytes 16*(l%8) .. +15 of the panel), written to the
// wave's LDS slot, and read back k-contiguous with ds_read_b64_tr_b8: within
// each 16-lane group, lane 2t supplies bytes 0..7 and lane 2t+1 bytes 8..15
// of row t, and lane i receives column i of the 8 x 16 byte block.  The 16
// byte chunks of a row are XOR-swizzled with the row index so that the eight
// rows of one transposed read fall into different LDS banks.
struct RawL {
  v4i a;
  v4i bq[4];
};

constexpr int kSlotBytes = kTile * kPanel;  // 4 KB: one B slab

// live == false (a batch slot past the item's end): every lane reads the
// same 16 bytes, so the slot costs one cache line but keeps the number of
// outstanding loads fixed, which lets the compiler's vmcnt waits stay exact.
template <int ELT>
__device__ __forceinline__ void load_raw_lds(const Params& p, int t, int kb, bool live, int j, int g,
                                             int lane, int panel_col, RawL& f) {
  // Offsets are masked arithmetically (not selected) so that the compiler
  // keeps these loads unconditional.
  const int64_t m = -(int64_t)live;
  f.a = *reinterpret_cast<const v4i*>(p.tiles + (((int64_t)t * (kTile * kTile) + j * kTile + g * 16) & m));
  const int chunk_col = panel_col + 16 * (lane & 7);
  const int col = chunk_col < p.N ? chunk_col : 0;  // past N: any valid chunk, never stored
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int k = kb * kTile + 8 * q + (lane >> 3);
    const int kc = k < p.K ? k : p.K - 1;
    f.bq[q] = *reinterpret_cast<const v4i*>(p.b + (((int64_t)kc * p.ldb + col) & m));
  }
}

template <int ELT>
__device__ __forceinline__ void stage_lds(const RawL& f, int kb, int K, int lane, uint8_t* slot) {
  const int kmax = K - kb * kTile;  // rows of the slab inside K
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int rowl = 8 * q + (lane >> 3);
    v4i v = f.bq[q];
    if (ELT == kEltFp8 && rowl >= kmax) v = v4i{0, 0, 0, 0};  // rows past K: fp8 codes may be NaN
    *reinterpret_cast<v4i*>(slot + rowl * kPanel + ((((lane & 7) ^ (rowl & 7))) << 4)) = v;
  }
}

__device__ __forceinline__ v4i read_tr(const uint8_t* slot, int c, int j, int g) {
  const int i = j & 15;
  const int s = 2 * c + (j >> 4);
  v4i out;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int rowl = 16 * g + 8 * h + (i >> 1);
    const uint8_t* a = slot + rowl * kPanel + ((s ^ (rowl & 7)) << 4) + 8 * (i & 1);
    typedef int v2i __attribute__((ext_vector_type(2)));
    const v2i v = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
        (__attribute__((address_space(3))) v2i*)(const_cast<uint8_t*>(a)));
    out[2 * h] = v[0];
    out[2 * h + 1] = v[1];
  }
  return out;
}

__device__ __forceinline__ float bcast(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// Row stride (dwords) of the LDS reduction buffer: 128 columns + 4 of padding
// keep the two row halves a wave writes in one instruction in different banks.
constexpr int kRedStride = kPanel + 32;  // also makes each wave's region hold kBatch B slabs

// Column position of (row, col) in the reduction buffer: rows 4 apart (the
// two halves of one MFMA result write) sit 16 banks apart.
__device__ __forceinline__ int red_col(int row, int col) { return col ^ (((row >> 2) & 1) << 4); }

template <int ELT, int EPI, int OUT, bool BCOL, bool VEC, bool LDSB>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) void spmm_bsr_kernel(Params p) {
  using A = Accum<ELT, EPI>;
  using Reg = typename A::Reg;
  constexpr bool kInt = A::kInt;

  // Per wave: 32 x 132 dwords of partial sums; during the tile loop the same
  // bytes hold the wave's kBatch B slabs (LDSB path).
  __shared__ __attribute__((aligned(16))) int red[kWaves][kTile][kRedStride];
  int& s_last = red[0][0][kPanel];  // padding word: split-row arrival flag
  static_assert(kBatch * kSlotBytes <= (int)sizeof(red[0]), "B slabs must fit the wave's LDS region");

  TRACE_DECL;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int j = lane & 31, g = lane >> 5;

  int item_idx, panel;
  if (!wg_map(p, item_idx, panel)) return;
  const void_work_item* itp = p.items + item_idx;
  // Block columns of the first batch (tiles wave + 4u, u < 4) through the
  // scalar cache, issued together with the record's fields: a cold scalar
  // load returns well before a cold vector load.
  const v4i* colv = reinterpret_cast<const v4i*>(itp->cols);
  const v4i cq0 = colv[0], cq1 = colv[1], cq2 = colv[2], cq3 = colv[3], cq4 = colv[4];
  __builtin_amdgcn_sched_barrier(0);
  const int row = itp->row, begin = itp->begin, end = itp->end, split_tile = itp->tile;
  const int col0 = panel * kPanel + j * kColsPerLane;
  (void)(row + begin + end);
  TRACE_POINT(0);

  // Load order matters: vmcnt retires vector loads in issue order, so a
  // value is usable only once every load issued before it has returned.
  // (1) the first batch's block columns (from the item record, lanes <
  //     kInline) and per-tile scales, (2) the first batch's A and B tiles,
  // (3) what is needed later: columns of further tiles, B scales, bias and
  //     the row-mean scales.
  // Tiles of the item are taken round-robin by the waves (wave w: tiles w,
  // w+4, ...); columns past the item's end are -1 and are clamped to a
  // valid address, their products skipped.
  const int nt = end - begin;
  const int tl = begin + min(lane, max(nt - 1, 0));
  float my_scale = 0.f;
  if constexpr (EPI == VOID_EPI_PER_BLOCK) {
    const float* msp = nt > 0 ? p.a_scale : reinterpret_cast<const float*>(p.row_ptr);  // empty: a dummy read
    my_scale = msp[nt > 0 && !p.per_tensor_a ? tl : 0];
  }
  auto scale_of = [&](int idx) -> float {
    if constexpr (EPI != VOID_EPI_PER_BLOCK) return 0.f;
    if (idx < 64) return bcast(my_scale, idx);
    return p.per_tensor_a ? p.a_scale[0] : p.a_scale[begin + idx];
  };

  Reg acc[kColsPerLane];
#pragma unroll
  for (int c = 0; c < kColsPerLane; ++c) acc[c] = Reg{};

  const int col_64 = nt > 0 ? p.col_idx[tl] : 0;  // before the tile loads: vmcnt retires in order
  const bool has_first = wave < nt;
  const v4i cq[5] = {cq0, cq1, cq2, cq3, cq4};
  static_assert(kBatch <= 5 && kBatch * kWaves <= kInline, "first batch columns come from the record");
  int kbs0[kBatch];
#pragma unroll
  for (int u = 0; u < kBatch; ++u)
    kbs0[u] = max(wave == 0 ? cq[u][0] : wave == 1 ? cq[u][1] : wave == 2 ? cq[u][2] : cq[u][3], 0);

  // Operand loading differs by B layout; everything else is shared.
  using RawT = typename std::conditional<LDSB, RawL, Raw>::type;
  uint8_t* stage = reinterpret_cast<uint8_t*>(&red[wave][0][0]);
  auto issue = [&](RawT& r, int idx, int kb) {
    const bool live = idx < nt;
    const int t = begin + (live ? idx : 0);
    if constexpr (LDSB) load_raw_lds<ELT>(p, t, live ? kb : 0, live, j, g, lane, panel * kPanel, r);
    else load_raw<BCOL, VEC>(p, t, live ? kb : 0, j, g, col0, r);
  };
  auto consume = [&](const RawT& r, int kb, int u, int idx, float sc) {
    Frag f;
    if constexpr (LDSB) {
      uint8_t* slot = stage + u * kSlotBytes;
      stage_lds<ELT>(r, kb, p.K, lane, slot);
      f.a = r.a;
#pragma unroll
      for (int c = 0; c < kColsPerLane; ++c) f.b[c] = read_tr(slot, c, j, g);
    } else {
      to_frag<ELT, BCOL>(r, f);
    }
    A::step(acc, f, sc);
  };

  RawT raw0[kBatch];
  if (has_first) {
#pragma unroll
    for (int u = 0; u < kBatch; ++u) issue(raw0[u], wave + u * kWaves, kbs0[u]);
  }
  TRACE_POINT(1);

  // Epilogue inputs, issued after the first tiles' loads.
  // Branch-free (a load under a branch would make the vmcnt waits above
  // conservative): absent vectors read a_scale[0] and are then ignored.
  float sb[4], bias[4];
  {
    const float* sbp = p.b_scale_vec ? p.b_scale_vec : reinterpret_cast<const float*>(p.row_ptr);
    const float* bip = p.bias ? p.bias : reinterpret_cast<const float*>(p.row_ptr);
    const int cmax = (p.b_scale_vec || p.bias) ? p.N - 1 : 0;
    float vs[4], vb[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int cc = min(col0 + c, cmax);
      vs[c] = sbp[p.b_scale_vec ? cc : 0];
      vb[c] = bip[p.bias ? cc : 0];
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      sb[c] = p.b_scale_vec ? vs[c] : p.b_scale;
      bias[c] = p.bias ? vb[c] : 0.f;
    }
  }
  int rb = 0, re = 0;
  float row_scale = 0.f;  // a_scale of the row's first 64 tiles, one per lane (row-mean)
  if constexpr (EPI == VOID_EPI_ROW_MEAN) {
    // An unsplit item is its whole block-row; a split row needs row_ptr.
    if (split_tile < 0) {
      rb = begin;
      re = end;
    } else {
      rb = p.row_ptr[row];
      re = p.row_ptr[row + 1];
    }
    // An empty row reads row_ptr[0] (always present) and ignores it.
    const float* rsp = re > rb ? p.a_scale : reinterpret_cast<const float*>(p.row_ptr);
    row_scale = rsp[re > rb ? (p.per_tensor_a ? 0 : rb + min(lane, re - rb - 1)) : 0];
  }

  if (has_first) {
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int idx = wave + u * kWaves;
      // idx < kBatch * kWaves < 64: the scale comes from my_scale without the
      // branch of scale_of (a branch here would blur the compiler's vmcnt count).
      if (idx < nt) consume(raw0[u], kbs0[u], u, idx, EPI == VOID_EPI_PER_BLOCK ? bcast(my_scale, idx) : 0.f);
    }
  }
  // Further rounds (items longer than kBatch * kWaves tiles).
  for (int base = wave + kBatch * kWaves; base < nt; base += kBatch * kWaves) {
    int kbs[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int idx = base + u * kWaves;
      const int ii = idx < nt ? idx : base;  // empty slots reload a valid tile and are skipped
      kbs[u] = ii < 64 ? __builtin_amdgcn_readlane(col_64, ii) : p.col_idx[begin + ii];
    }
    RawT raw[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) issue(raw[u], base + u * kWaves, kbs[u]);
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int idx = base + u * kWaves;
      if (idx < nt) consume(raw[u], kbs[u], u, idx, scale_of(idx));
    }
  }

  TRACE_POINT(2);

  // Cross-wave reduction.  MFMA 32x32 result layout: lane l, register r holds
  // row 8*(r/4) + 4*(l/32) + r%4 of virtual column l%32.
  // LDSB: MFMA c holds columns 32c + j; otherwise columns 4j + c.
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int rr = 8 * (r >> 2) + 4 * g + (r & 3);
    if constexpr (LDSB) {
#pragma unroll
      for (int c = 0; c < kColsPerLane; ++c)
        red[wave][rr][red_col(rr, 32 * c + j)] = kInt ? (int)acc[c][r] : __float_as_int((float)acc[c][r]);
    } else {
      v4i w;
#pragma unroll
      for (int c = 0; c < kColsPerLane; ++c) w[c] = kInt ? (int)acc[c][r] : __float_as_int((float)acc[c][r]);
      *reinterpret_cast<v4i*>(&red[wave][rr][red_col(rr, 4 * j)]) = w;
    }
  }
  __syncthreads();

  // Epilogue ownership: wave w finishes rows [8w, 8w+8); lane owns columns
  // col0 .. col0+3 (same j as above) of rows 8w + g + 2i.
  v4i sumi[kRowsPerWave / 2];
  v4f sumf[kRowsPerWave / 2];
#pragma unroll
  for (int i = 0; i < kRowsPerWave / 2; ++i) {
    const int rr = wave * kRowsPerWave + 2 * i + g;
    v4i si = {0, 0, 0, 0};
    v4f sf = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const v4i x = *reinterpret_cast<const v4i*>(&red[w][rr][red_col(rr, 4 * j)]);
      if constexpr (kInt) si += x;
      else sf += v4f{__int_as_float(x[0]), __int_as_float(x[1]), __int_as_float(x[2]), __int_as_float(x[3])};
    }
    sumi[i] = si;
    sumf[i] = sf;
  }
  TRACE_POINT(3);

  if (itp->tile >= 0) {
    // Split row: publish this chunk's partial tile with agent-coherent (sc1)
    // stores, count arrivals, and let the last chunk read every partial back
    // with agent-coherent loads and reduce them in chunk order.  Coherent
    // accesses replace release/acquire fences, which would write back and
    // invalidate the whole L2 of the XCD.
    const int tile_id = itp->tile, nchunks = itp->nchunks, slot = itp->slot, chunk = itp->chunk;
    const size_t tile_elems = (size_t)kTile * kPanel;
    int* part = static_cast<int*>(p.partials);
#pragma unroll
    for (int i = 0; i < kRowsPerWave / 2; ++i) {
      const int rr = wave * kRowsPerWave + 2 * i + g;
      const size_t off = ((size_t)(slot + chunk) * p.n_panels + panel) * tile_elems + (size_t)rr * kPanel + 4 * j;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int w = kInt ? sumi[i][c] : __float_as_int(sumf[i][c]);
        __hip_atomic_store(part + off + c, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    publish_wait();  // this wave's partial stores are acknowledged
    __syncthreads();
    unsigned* ctr = p.counters + (size_t)tile_id * p.n_panels + panel;
    if (tid == 0) {
      const unsigned old = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      s_last = (old == (unsigned)(nchunks - 1));
    }
    __syncthreads();
    if (!s_last) {
      TRACE_FLUSH();
      return;
    }
    if (tid == 0) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    compiler_order();  // the partial loads stay below the arrival count
#pragma unroll
    for (int i = 0; i < kRowsPerWave / 2; ++i) {
      const int rr = wave * kRowsPerWave + 2 * i + g;
      v4i si = {0, 0, 0, 0};
      v4f sf = {0.f, 0.f, 0.f, 0.f};
      for (int ch = 0; ch < nchunks; ++ch) {
        const size_t off = ((size_t)(slot + ch) * p.n_panels + panel) * tile_elems + (size_t)rr * kPanel + 4 * j;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const int x = __hip_atomic_load(part + off + c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          if constexpr (kInt) si[c] += x;
          else sf[c] += __int_as_float(x);
        }
      }
      sumi[i] = si;
      sumf[i] = sf;
    }
  }

  float mul[4] = {1.f, 1.f, 1.f, 1.f};
  if constexpr (EPI == VOID_EPI_ROW_MEAN) {
    // int_quant.py:519-526: S = sum fl(s_a * s_b) in tile order over the
    // whole block-row, then S / n.  The row's scales sit one per lane and
    // are folded sequentially with readlane.
    float S[4] = {0.f, 0.f, 0.f, 0.f};
    for (int t0 = rb; t0 < re; t0 += 64) {
      const int n = min(64, re - t0);
      const float mine = t0 == rb ? row_scale
                                  : (p.per_tensor_a ? p.a_scale[0] : p.a_scale[t0 + min(lane, n - 1)]);
      for (int q = 0; q < n; ++q) {
        const float sa = bcast(mine, q);
#pragma unroll
        for (int c = 0; c < 4; ++c) S[c] = __fadd_rn(S[c], __fmul_rn(sa, sb[c]));
      }
    }
    const float n = (float)(re - rb);
#pragma unroll
    for (int c = 0; c < 4; ++c) mul[c] = (re > rb) ? __fdiv_rn(S[c], n) : 0.f;
  } else if constexpr (EPI == VOID_EPI_PER_BLOCK) {
#pragma unroll
    for (int c = 0; c < 4; ++c) mul[c] = sb[c];
  }

#pragma unroll
  for (int i = 0; i < kRowsPerWave / 2; ++i) {
    const int rr = wave * kRowsPerWave + 2 * i + g;
    const int grow = row * kTile + rr;
    float v[4];
    int vi[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      vi[c] = sumi[i][c];
      float x;
      if constexpr (EPI == VOID_EPI_ROW_MEAN) x = __fmul_rn((float)sumi[i][c], mul[c]);
      else if constexpr (EPI == VOID_EPI_PER_BLOCK) x = __fmul_rn(sumf[i][c], mul[c]);
      else x = 0.f;
      if (p.bias) x = __fadd_rn(x, bias[c]);
      v[c] = activate(x, p.activation);
    }
    store4<OUT, VEC>(p, grow, col0, v, vi);
  }
  TRACE_POINT(4);
  TRACE_FLUSH();
}

// ---------------------------------------------------------------------------
// Host side

thread_local char g_err[512];

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof g_err, fmt, ap);
  va_end(ap);
  return code;
}

}  // namespace

// Error reporting for the library's other translation units.
extern "C" __attribute__((visibility("hidden"))) int void_internal_fail(int code, const char* msg) {
  return fail(code, "%s", msg);
}

namespace {

template <int ELT, int EPI, int OUT, bool BCOL, bool VEC, bool LDSB = false>
int launch(const Params& p, int grid, hipStream_t stream) {
  hipLaunchKernelGGL((spmm_bsr_kernel<ELT, EPI, OUT, BCOL, VEC, LDSB>), dim3(grid), dim3(kThreads), 0, stream, p);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(VOID_ERR_HIP, "kernel launch failed: %s", hipGetErrorString(e));
  return VOID_OK;
}

// ---------------------------------------------------------------------------
// Column-group kernel: row-major B with 16-byte aligned rows, or
// column-major B with K % 32 == 0.
//
// One workgroup = 4 wave64s = one work item x one 128-column panel, as for
// spmm_bsr_kernel, but every wave runs all of the item's tiles for its own 32
// output columns (column group cg = 4 * panel + wave), so no cross-wave
// reduction is needed.  Tiles go in batches of kCgBatch, staged through a
// double-buffered LDS area with one barrier per batch:
//  - A: each wave loads two of the batch's tiles (MFMA fragment order);
//  - row-major B: each wave loads 8 of the 32 rows of every tile's
//    32 x 128 slab (full 128-byte lines), written with the same XOR chunk
//    swizzle as stage_lds; every wave then reads its own 32 columns back
//    k-contiguous with ds_read_b64_tr_b8 (read_tr);
//  - column-major B: each wave loads its MFMA operands directly.
// The loads of batch b + 1 are in flight while batch b is multiplied, and
// every tile-dependent address is a wave-uniform buffer offset (SGPR), so
// the tile loop spends no vector ALU work on addressing.
// A work item has at most kCgMaxTiles tiles: the block columns of batches 0
// and 1 come with the work item, the rest and the per-tile scales are one
// dword per lane of a single load issued before the first batch.
constexpr int kCgBatch = 8;
constexpr int kCgAPerWave = kCgBatch / kWaves;
constexpr int kCgMaxTiles = 64;
static_assert(2 * kCgBatch <= kInline, "the first two batches' columns come from the work item");

typedef __amdgpu_buffer_rsrc_t Rsrc;

// Raw buffers (stride 0) span 2^31 - 1 bytes; the host checks that every
// operand's offsets fit in 31 bits.  Slots past the end of an item are
// filled by loads at kOutOfRange (zeros, no memory request), so that the
// number of issued loads (and so every vmcnt wait) stays fixed.

__device__ __forceinline__ Rsrc make_rsrc(const void* p) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, 0x7fffffff, 0x00020000);
}

// One tile's MFMA operands for a single 32-column group.
struct Frag1 {
  v4i a;
  v4i b;
};

template <int ELT, int EPI>
struct Accum1;

template <int EPI>
struct Accum1<kEltI8, EPI> {
  static constexpr bool kInt = (EPI != VOID_EPI_PER_BLOCK);
  using Reg = typename std::conditional<kInt, v16i, v16f>::type;
  using Part = v16i;
  // Per-block epilogue split in two, so that products of several tiles can
  // be in flight before their scaled adds.
  __device__ __forceinline__ static Part prod(const Frag1& f) {
    const v16i z = {};
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(f.a, f.b, z, 0, 0, 0);
  }
  __device__ __forceinline__ static void fold(Reg& acc, const Part& part, float s) {
    if constexpr (!kInt) {
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[r] = __builtin_fmaf(s, (float)part[r], acc[r]);
    }
  }
  __device__ __forceinline__ static void step(Reg& acc, const Frag1& f, float s) {
    if constexpr (kInt) {
      acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(f.a, f.b, acc, 0, 0, 0);
    } else {
      const v16i z = {};
      const v16i part = __builtin_amdgcn_mfma_i32_32x32x32_i8(f.a, f.b, z, 0, 0, 0);
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[r] = __builtin_fmaf(s, (float)part[r], acc[r]);
    }
  }
};

template <int EPI>
struct Accum1<kEltFp8, EPI> {
  static constexpr bool kInt = false;
  using Reg = v16f;
  using Part = v16f;
  __device__ __forceinline__ static Part prod(const Frag1& f) {
    const v16f z = {};
    v16f part = __builtin_amdgcn_mfma_f32_32x32x16_fp8_fp8(pack2(f.a[0], f.a[1]), pack2(f.b[0], f.b[1]), z, 0, 0, 0);
    return __builtin_amdgcn_mfma_f32_32x32x16_fp8_fp8(pack2(f.a[2], f.a[3]), pack2(f.b[2], f.b[3]), part, 0, 0, 0);
  }
  __device__ __forceinline__ static void fold(Reg& acc, const Part& part, float s) {
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = __builtin_fmaf(s, part[r], acc[r]);
  }
  __device__ __forceinline__ static void step(Reg& acc, const Frag1& f, float s) {
    const v16f z = {};
    v16f part = __builtin_amdgcn_mfma_f32_32x32x16_fp8_fp8(pack2(f.a[0], f.a[1]), pack2(f.b[0], f.b[1]), z, 0, 0, 0);
    part = __builtin_amdgcn_mfma_f32_32x32x16_fp8_fp8(pack2(f.a[2], f.a[3]), pack2(f.b[2], f.b[3]), part, 0, 0, 0);
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = __builtin_fmaf(s, part[r], acc[r]);
  }
};

// fp32 tiles (float SpMM): fp32 accumulation, no per-tile scales.
template <int EPI>
struct Accum1<kEltF32, EPI> {
  static constexpr bool kInt = false;
  using Reg = v16f;
  using Part = v16f;
  // Never called: the fp32 tile product is written out in the ring loop; the
  // register-staged loop that names these is not used for fp32 tiles.
  __device__ __forceinline__ static void step(Reg&, const Frag1&, float) {}
  __device__ __forceinline__ static Part prod(const Frag1&) { return Part{}; }
  __device__ __forceinline__ static void fold(Reg&, const Part&, float) {}
};

// E4M3 tiles times fp32 B: fp32 accumulation, per-tile scales applied in the
// ring loop (which computes this product itself, like the fp32 tiles').
template <int EPI>
struct Accum1<kEltFp8F32, EPI> : Accum1<kEltF32, EPI> {};

// bf16 / fp16 tiles: fp32 accumulation, no per-tile scales, product in the
// ring loop.
template <int EPI>
struct Accum1<kEltBf16, EPI> : Accum1<kEltF32, EPI> {};
template <int EPI>
struct Accum1<kEltF16, EPI> : Accum1<kEltF32, EPI> {};
// E4M3 tiles times a 16-bit B: as E4M3 times fp32 B.
template <int EPI>
struct Accum1<kEltFp8Bf16, EPI> : Accum1<kEltF32, EPI> {};
template <int EPI>
struct Accum1<kEltFp8F16, EPI> : Accum1<kEltF32, EPI> {};

typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef _Float16 v8hf __attribute__((ext_vector_type(8)));
typedef __bf16 v2bf __attribute__((ext_vector_type(2)));

// Two floats rounded to bf16 (nearest even, v_cvt_pk_bf16_f32), packed.
__device__ __forceinline__ uint32_t pack_bf16_rne(float x0, float x1) {
  const v2bf h = {(__bf16)x0, (__bf16)x1};
  return __builtin_bit_cast(uint32_t, h);
}

// The upper halves of two floats (bf16 by truncation), packed.
__device__ __forceinline__ uint32_t pack_bf16_trunc(float x0, float x1) {
  return __builtin_amdgcn_perm(__float_as_uint(x1), __float_as_uint(x0), 0x07060302u);
}

// Four E4M3FN codes (one dword, code i in byte i) -> four bf16 values in two
// dwords.  Every E4M3 value (subnormals included; the NaN codes stay NaN) is
// exact in fp32 and in bf16 (3 mantissa bits, exponents 2^-9 .. 2^8), so the
// truncating pack is exact.
__device__ __forceinline__ void e4m3x4_to_bf16(uint32_t w, uint32_t& lo, uint32_t& hi) {
  const v2f f01 = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, false);
  const v2f f23 = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, true);
  lo = pack_bf16_trunc(f01[0], f01[1]);
  hi = pack_bf16_trunc(f23[0], f23[1]);
}

// The same to fp16 (also exact: E4M3's values, subnormals included, lie in
// fp16's normal range with at most 4 significant bits).
__device__ __forceinline__ void e4m3x4_to_f16(uint32_t w, uint32_t& lo, uint32_t& hi) {
  const v2f f01 = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, false);
  const v2f f23 = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, true);
  lo = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(f01[0], f01[1]));
  hi = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(f23[0], f23[1]));
}

// Split of fp32 x into bf16 hi + lo: hi = x truncated to bf16 (x - hi is then
// exact in fp32 and below 2^-7 |x|), lo = bf16(x - hi) to nearest, so that
// |x - hi - lo| <= 2^-16 |x| (short of bf16's normal range, x below about
// 2^-118, lo loses bits).  Two values per call, packed.
__device__ __forceinline__ void split_bf16(float x0, float x1, uint32_t& hi, uint32_t& lo) {
  hi = pack_bf16_trunc(x0, x1);
  const float r0 = x0 - __uint_as_float(__float_as_uint(x0) & 0xffff0000u);
  const float r1 = x1 - __uint_as_float(__float_as_uint(x1) & 0xffff0000u);
  lo = pack_bf16_rne(r0, r1);
}

struct CgBatch {
  v4i a[kCgAPerWave];  // A tiles wave + 4q of the batch, lane (j, g): row j, bytes 16g .. 16g+15
  v4i b[kCgBatch];     // row-major B: slab row 8 wave + lane / 8, bytes 16 (lane % 8) .. +15;
                       // column-major B: the MFMA operand (column j, rows 16g .. 16g+15)
  int last_mask;       // bit u: tile u's slab is the one that crosses K
};

// LDS-DMA variant (DMA = true, row-major B only): the same work split, but
// the tile slots form a ring of kDmaStages stages of kDmaTiles tiles, filled
// by buffer loads that write LDS directly (buffer_load_dwordx4 ... lds), so
// no batch is staged in registers.  Two stages (40 KB) and about 100 VGPRs
// let four workgroups (16 waves) share a CU; one workgroup's record fetch,
// stage waits and epilogue then overlap the others' MFMA work.  Measured
// against deeper rings at lower occupancy (4 stages with 2 workgroups per
// CU, 2-tile stages with 4-6 workgroups), this was fastest on c2, c3 and c5.
// A wave issues kDmaTiles B loads per stage (8 rows of each slab), and the
// first kDmaTiles waves one A tile each, so the wait for stage s is vmcnt of
// that count times the stages issued after s.
constexpr int kDmaTiles = 4;
constexpr int kDmaStages = 2;
constexpr int kDmaWavesPerEu = 4;  // workgroups per CU, as LDS (4 x 40 KB) allows
// The 3-tile ring: 3 tiles per stage (30 KB), 5 workgroups per CU.  On
// grids beyond one resident round the extra waves hide more of each
// workgroup's start and epilogue (c5: 91 -> 87 us; 1024-4096 workgroup
// uniform grids: 2-5 % over the 4-tile ring); on one-round grids the
// shallower stages lose (c3: 11.5 -> 12.6 us).
constexpr int kDmaTilesDeep = 3;
constexpr int kDeepGridRounds = 4;  // split plans of at least this many 1024-workgroup rounds take it
constexpr int kPairGridMax = 512;   // two-ring (8-wave, 80 KB) workgroups: 2 per CU, one round
__host__ __device__ constexpr int dma_waves_per_eu(int tiles) { return tiles == kDmaTilesDeep ? 5 : kDmaWavesPerEu; }
static_assert(kDmaTiles <= kWaves && kDmaTilesDeep <= kWaves, "at most one A tile per wave per stage");
static_assert(kDmaStages >= 2 && kDmaStages <= 4, "stage waits cover up to two stages ahead");

// Cache policy of the staged C stores: nt | sc1 (non-temporal, agent
// scope).  C is written once and not read by the kernel; on c2 this measured
// 8.7 us cold / 7.2 us hot against 9.2-9.3 / 8.0 with the default policy
// (on the later two-ring kernel nt, sc0 | nt, sc0 | sc1 and sc0 | sc1 | nt
// all measured within noise of it on c2, c3 and c5).
constexpr int kStoreStream = 2 | 16;

// LDS-DMA loads, their SGPR descriptors and the ring's waits: lds_dma.h.

template <int ELT, int EPI, int OUT, bool BCOL, bool DMA = false, int RT = kDmaTiles, int KS = 1>
__global__ __launch_bounds__(kThreads * KS) __attribute__((amdgpu_waves_per_eu(
    DMA ? (KS > 1 ? 4 : dma_waves_per_eu(RT)) : 2, DMA ? (KS > 1 ? 4 : dma_waves_per_eu(RT)) : 2))) void
    spmm_cg_kernel(const void_work_item* __restrict__ items, int map_word, int map_items, int map_panels, Params p) {
  static_assert(!(DMA && BCOL), "the LDS-DMA ring is for row-major B");
  static_assert(KS == 1 || (DMA && KS == 2), "the two-ring split is for the LDS-DMA ring");
  using A = Accum1<ELT, EPI>;
  constexpr bool kInt = A::kInt;
  constexpr bool kF32 = ELT == kEltF32;                     // fp32 A tiles
  constexpr bool kBF32 = kF32 || ELT == kEltFp8F32;         // fp32 B slabs
  constexpr bool k16 = ELT == kEltBf16 || ELT == kEltF16;   // 16-bit tiles and B
  constexpr bool kF8B16 = ELT == kEltFp8Bf16 || ELT == kEltFp8F16;  // E4M3 tiles, 16-bit B
  constexpr bool kB16 = k16 || kF8B16;                      // 16-bit B slabs
  constexpr bool kFloat = kF32 || k16;                      // unscaled float tiles
  static_assert(!(kBF32 || kB16) || DMA, "fp32 and 16-bit B only on the LDS-DMA ring");
  constexpr bool kScales = (EPI == VOID_EPI_PER_BLOCK) && !kFloat;
  // fp32 B: 4 bytes per element, one tile per stage (a 16 KB B slab, and 4 KB
  // of A for fp32 tiles or 1 KB for E4M3 ones); 16-bit: two tiles per stage
  // (8 KB slab + 2 KB tile each).  Either way the ring keeps its 40 KB.
  constexpr int kEsz = kF32 ? 4 : k16 ? 2 : 1;    // A
  constexpr int kBEsz = kBF32 ? 4 : kB16 ? 2 : 1;  // B
  constexpr int kStageTiles = kBF32 ? 1 : kB16 ? 2 : RT;

  // Tile slots: two batches of the register-staged loop, or the LDS-DMA ring.
  // KS = 2: two groups of 4 waves, each with its own ring, take alternate
  // stages of the same item and add their accumulators at the end.
  constexpr int kSlots = DMA ? kDmaStages * kStageTiles : 2 * kCgBatch;
  __shared__ __attribute__((aligned(16))) v4i a_lds[KS * kSlots][64 * kEsz];
  __shared__ __attribute__((aligned(16))) uint8_t b_lds[BCOL ? 1 : KS * kSlots][BCOL ? 16 : kSlotBytes * kBEsz];
  // Split-row arrival flag: the first word of the A area, free once every
  // wave has passed the tile loop (no LDS word is spare: 80 KB keeps the
  // register-staged loop at two workgroups per CU, 40 KB the ring at four).
  int& s_last = *reinterpret_cast<int*>(&a_lds[0][0]);

  TRACE_DECL;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane((tid >> 6) & (kWaves - 1));
  const int sg = KS > 1 ? __builtin_amdgcn_readfirstlane(tid >> 8) : 0;  // wave group
  const int lane = tid & 63;
  const int j = lane & 31, g = lane >> 5;

  int item_idx, panel;
  if (!wg_map_args(map_word, map_items, map_panels, item_idx, panel)) return;
  const void_work_item* itp = items + item_idx;
  const v4i* colv = reinterpret_cast<const v4i*>(itp->cols);
  const v4i cq0 = colv[0], cq1 = colv[1], cq2 = colv[2], cq3 = colv[3];
  __builtin_amdgcn_sched_barrier(0);
  const int row = itp->row, begin = itp->begin, end = itp->end, split_tile = itp->tile;
  const int nt = end - begin;
  const int cg = panel * kWaves + wave;
  const int col = cg * kTile + j;  // this lane's output column
  TRACE_POINT(0);
  TRACE_TAG((unsigned long long)nt | ((unsigned long long)blockIdx.x << 16));

  const Rsrc ra = make_rsrc(p.tiles), rbm = make_rsrc(p.b), rcol = make_rsrc(p.col_idx),
             rsc = make_rsrc(p.a_scale);
  // Per-lane parts of the operand offsets, fixed for the whole item.
  const int voff_a = j * kTile + 16 * g;
  int voff_b, voff_b_last = 0, kb_last = -1;
  const int brow = 8 * wave + (lane >> 3);  // row-major: this lane's slab row
  if constexpr (BCOL) {
    const int cc = col < p.N ? col : 0;  // past N: any valid column, never stored
    voff_b = (int)(cc * p.ldb) + 16 * g;
  } else {
    int cb = panel * kPanel + 16 * (lane & 7);
    cb = cb < p.N ? cb : 0;  // past N: any valid 16 bytes, never stored
    voff_b = (int)(brow * p.ldb) + cb;
    if (p.K % kTile) {  // the last slab reads row K-1 in place of rows past K
      kb_last = p.K / kTile;
      voff_b_last = (int)(min(brow, p.K - kb_last * kTile - 1) * p.ldb) + cb;
    }
  }
  const int b_kstride = BCOL ? kTile : kTile * (int)p.ldb * kBEsz;  // bytes per block column

  // Epilogue inputs, issued before the tile loads (branch-free: a load under
  // a branch would make the compiler's vmcnt waits conservative).
  float sb, bias;
  {
    const float* sbp = p.b_scale_vec ? p.b_scale_vec : reinterpret_cast<const float*>(p.row_ptr);
    const float* bip = p.bias ? p.bias : reinterpret_cast<const float*>(p.row_ptr);
    const int cc = min(col, p.N - 1);
    const float vs = sbp[p.b_scale_vec ? cc : 0];
    const float vb = bip[p.bias && !p.bias_per_row ? cc : 0];  // a per-row bias has M entries
    sb = p.b_scale_vec ? vs : p.b_scale;
    bias = p.bias ? vb : 0.f;
  }
  int rb = 0, re = 0;
  float row_scale = 0.f;  // row-mean: a_scale of the row's first 64 tiles, one per lane
  if constexpr (EPI == VOID_EPI_ROW_MEAN) {
    if (split_tile < 0) {
      rb = begin;
      re = end;
    } else {
      rb = p.row_ptr[row];
      re = p.row_ptr[row + 1];
    }
    // An empty row reads row_ptr[0] (always present) and ignores it.
    const float* rsp = re > rb ? p.a_scale : reinterpret_cast<const float*>(p.row_ptr);
    row_scale = rsp[re > rb ? (p.per_tensor_a ? 0 : rb + min(lane, re - rb - 1)) : 0];
  }

  typename A::Reg acc = {};
  int kbs[kCgBatch];
  int colw = 0;      // lane i: block column of tile min(i, nt - 1)
  float scw = 0.f;   // lane i: a_scale of that tile (per-block epilogues)
  // Block columns of batch bb: batches 0 and 1 from the work item (-1 marks
  // slots past the item's end; they re-read the first column), later ones
  // from colw (slots past the end read tile nt - 1's column).
  auto take_cols = [&](int bb) {
#pragma unroll
    for (int u = 0; u < kCgBatch; ++u) {
      int kb;
      if (bb < 2) {
        const int c0 = u < 4 ? cq0[u & 3] : cq1[u & 3];
        const int c1 = u < 4 ? cq2[u & 3] : cq3[u & 3];
        kb = bb == 0 ? c0 : c1;
        kb = kb >= 0 ? kb : max(cq0[0], 0);
      } else {
        kb = __builtin_amdgcn_readlane(colw, min(bb * kCgBatch + u, kCgMaxTiles - 1));
      }
      kbs[u] = __builtin_amdgcn_readfirstlane(kb);
    }
  };
  auto issue = [&](CgBatch& x, int bb) {
    const int base = bb * kCgBatch;
#pragma unroll
    for (int q = 0; q < kCgAPerWave; ++q) {
      const int idx = base + wave + kWaves * q;
      const bool live = idx < nt;
      x.a[q] = __builtin_amdgcn_raw_buffer_load_b128(ra, live ? voff_a : kOutOfRange,
                                                     (begin + (live ? idx : 0)) * (kTile * kTile), 0);
    }
    int mask = 0;
#pragma unroll
    for (int u = 0; u < kCgBatch; ++u) {
      int vo = voff_b;
      if constexpr (!BCOL) {
        const bool last = kbs[u] == kb_last;
        mask |= (int)last << u;
        vo = last ? voff_b_last : voff_b;
      }
      x.b[u] = __builtin_amdgcn_raw_buffer_load_b128(rbm, base + u < nt ? vo : kOutOfRange, kbs[u] * b_kstride, 0);
    }
    x.last_mask = mask;
  };
  auto consume = [&](const CgBatch& x, int bb) {
    const int base = bb * kCgBatch;
    const int buf = bb & 1;
#pragma unroll
    for (int q = 0; q < kCgAPerWave; ++q) a_lds[buf * kCgBatch + wave + kWaves * q][lane] = x.a[q];
    if constexpr (!BCOL) {
#pragma unroll
      for (int u = 0; u < kCgBatch; ++u) {
        v4i v = x.b[u];
        if constexpr (ELT == kEltFp8) {
          // Rows past K in the slab that crosses K: fp8 codes there may be
          // NaN, and NaN times the zero padding of A is still NaN.
          if (((x.last_mask >> u) & 1) && brow >= p.K - kb_last * kTile) v = v4i{0, 0, 0, 0};
        }
        *reinterpret_cast<v4i*>(&b_lds[buf * kCgBatch + u][brow * kPanel + (((lane & 7) ^ (brow & 7)) << 4)]) = v;
      }
    }
    __syncthreads();
#pragma unroll
    for (int u = 0; u < kCgBatch; ++u) {
      if (base + u < nt) {
        Frag1 f;
        f.a = a_lds[buf * kCgBatch + u][lane];
        if constexpr (BCOL) f.b = x.b[u];
        else f.b = read_tr(&b_lds[buf * kCgBatch + u][0], wave, j, g);
        float s = 0.f;
        if constexpr (kScales) s = bcast(scw, base + u);
        A::step(acc, f, s);
      }
    }
  };

  if constexpr (DMA) {
    v4i(*a_ring)[64 * kEsz] = a_lds + sg * kSlots;
    uint8_t(*b_ring)[kSlotBytes * kBEsz] = b_lds + sg * kSlots;
    const v4s da = sgpr_rsrc(p.tiles), db = sgpr_rsrc(p.b), dcol = sgpr_rsrc(p.col_idx), dsc = sgpr_rsrc(p.a_scale);
    // Each wave's own copy of the item's block columns and scales (one per
    // lane), parked in the B area of the last stage's first slot until the
    // first stage has landed: that slot is first refilled after the barrier
    // of stage 0, when every wave has read its copy back.
    int* win = reinterpret_cast<int*>(&b_ring[(kDmaStages - 1) * kStageTiles][wave * 512]);
    if (nt > 0) {
      const int ci = begin + min(lane, nt - 1);
      dma_b32(dcol, win, ci * 4, 0);
      if constexpr (kScales) dma_b32(dsc, win + 64, p.per_tensor_a ? 0 : ci * 4, 0);
    }
    // Lane (row brow, 16-byte position lane & 7) of a slab receives global
    // chunk (lane & 7) ^ (brow & 7): the XOR swizzle read_tr expects.  Rows
    // past K in the slab that crosses K load nothing (out of range).
    int cbd = panel * kPanel + 16 * ((lane & 7) ^ (brow & 7));
    cbd = cbd < p.N ? cbd : 0;  // past N: any valid 16 bytes, never stored
    const int voffd = (int)(brow * p.ldb) + cbd;
    const int voffd_last = (kb_last < 0 || brow < p.K - kb_last * kTile) ? voffd : kOutOfRange;
    // fp32: wave w fills rows 8 w .. 8 w + 7 of the slab (512 bytes each), two
    // rows per load; lane (row r, 16-byte position q) loads chunk q ^ 8 for
    // r >= 16, so that the two half waves of a column read use other banks.
    // A tile rows (128 bytes) take the 8-chunk swizzle q ^ (r & 7).
    int voffs_f[4] = {0, 0, 0, 0};
    int voff_af = 0;
    if constexpr (kBF32) {
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int r = 8 * wave + 2 * k + (lane >> 5);
        int cb = panel * kPanel * 4 + 16 * ((lane & 31) ^ (((r >> 4) & 1) << 3));
        cb = cb < p.N * 4 ? cb : 0;  // past N: any valid 16 bytes, never stored
        const int v = (int)(r * p.ldb * 4) + cb;
        voffs_f[k] = v;
      }
      const int ra_row = 8 * wave + (lane >> 3);
      voff_af = ra_row * (kTile * 4) + 16 * ((lane & 7) ^ (ra_row & 7));
    }
    auto voff_f_last = [&](int k) -> int {
      const int r = 8 * wave + 2 * k + (lane >> 5);
      return (kb_last < 0 || r < p.K - kb_last * kTile) ? voffs_f[k] : kOutOfRange;
    };
    // 16-bit B: a slab row is 256 bytes (16 chunks); wave w fills rows 8 w ..
    // 8 w + 7, four rows per load.  LDS chunk q of row r holds global chunk
    // q ^ ((r & 3) << 2), so the four rows of one transposed read sit in four
    // different bank quarters.  16-bit A: a tile is 32 rows of 64 bytes; wave
    // w loads half w & 1 (16 rows) of the stage's tile w >> 1, and LDS chunk
    // q of row r holds global chunk q ^ ((r >> 2) & 3).
    int voffs_h[2] = {0, 0}, voffs_h_last[2] = {0, 0};
    int voff_ah = 0;
    if constexpr (kB16) {
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        const int r = 8 * wave + 4 * k + (lane >> 4);
        int cb = panel * kPanel * 2 + 16 * ((lane & 15) ^ ((r & 3) << 2));
        cb = cb < p.N * 2 ? cb : 0;  // past N: any valid 16 bytes, never stored
        voffs_h[k] = (int)(r * p.ldb * 2) + cb;
        voffs_h_last[k] = (kb_last < 0 || r < p.K - kb_last * kTile) ? voffs_h[k] : kOutOfRange;
      }
      const int ar = 16 * (wave & 1) + (lane >> 2);
      voff_ah = ar * (kTile * 2) + 16 * ((lane & 3) ^ ((ar >> 2) & 3));
    }
    // Stages of the item; wave group sg takes global stages sg, sg + KS, ...
    // (ns of them), and both groups run ns_loop iterations so that they meet
    // at every barrier.
    const int ns_all = (nt + kStageTiles - 1) / kStageTiles;
    const int ns = (ns_all - sg + KS - 1) / KS;
    const int ns_loop = (ns_all + KS - 1) / KS;
    // The first RT waves also load one A tile per stage (wave 0 the one E4M3
    // tile of a stage with fp32 B; every wave a quarter of an fp32 tile).
    const bool a_wave = wave < (kBF32 ? 1 : k16 ? kWaves : kF8B16 ? 2 : RT);
    // Stages issued before the windows land (the prologue, s < kDmaStages - 1,
    // a constant after unrolling) read their columns from the work item
    // (tiles below 16); later ones from colw.
    static_assert((kDmaStages - 1) * KS * kDmaTiles <= 16, "prologue tiles come from the work item");
    auto stage_col = [&](int s, int u) -> int {
      const int t = (s * KS + sg) * kStageTiles + u;
      int kb;
      if (s < kDmaStages - 1) {
        // Selects, not a dynamic vector index (that would go through scratch).
        // Element first, then vector, on values (selecting a vector by a
        // run-time index made the compiler build a table in scratch).
        const int q = t >> 2, e = t & 3;
        auto el = [&](const v4i& c) { return e == 0 ? c[0] : e == 1 ? c[1] : e == 2 ? c[2] : c[3]; };
        const int k0 = el(cq0), k1 = el(cq1), k2 = el(cq2), k3 = el(cq3);
        kb = q == 0 ? k0 : q == 1 ? k1 : q == 2 ? k2 : k3;
        kb = kb >= 0 ? kb : max(cq0[0], 0);
      } else {
        kb = __builtin_amdgcn_readlane(colw, min(t, kCgMaxTiles - 1));
      }
      return __builtin_amdgcn_readfirstlane(kb);
    };
    auto issue_stage = [&](int s) {
      const int slot0 = (s % kDmaStages) * kStageTiles;
      const int base = (s * KS + sg) * kStageTiles;
      if constexpr (kB16) {
        // 16-bit tiles: one A load (half a tile) and four B loads per wave,
        // 5 per stage.  E4M3 tiles: waves 0 and 1 load one 1 KB tile each
        // (5 loads), the others only their four B loads.
        if constexpr (k16) {
          const int idx = base + (wave >> 1);
          const bool live = idx < nt;
          dma_b128(da, &a_ring[slot0 + (wave >> 1)][(wave & 1) * 64], live ? voff_ah : kOutOfRange,
                   (begin + (live ? idx : 0)) * (kTile * kTile * 2));
        } else if (a_wave) {
          const int idx = base + wave;
          const bool live = idx < nt;
          dma_b128(da, &a_ring[slot0 + wave][0], live ? voff_a : kOutOfRange, (begin + (live ? idx : 0)) * (kTile * kTile));
        }
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const int kb = stage_col(s, u);
          const bool live = base + u < nt;
#pragma unroll
          for (int k = 0; k < 2; ++k) {
            const int vo = live ? (kb == kb_last ? voffs_h_last[k] : voffs_h[k]) : kOutOfRange;
            dma_b128(db, &b_ring[slot0 + u][(8 * wave + 4 * k) * (kPanel * 2)], vo, kb * b_kstride);
          }
        }
        return;
      }
      if constexpr (kBF32) {
        const bool live = base < nt;
        if constexpr (kF32) {
          dma_b128(da, &a_ring[slot0][wave * 64], live ? voff_af : kOutOfRange,
                   (begin + (live ? base : 0)) * (kTile * kTile * 4));
        } else if (a_wave) {
          dma_b128(da, &a_ring[slot0][0], live ? voff_a : kOutOfRange, (begin + (live ? base : 0)) * (kTile * kTile));
        }
        const int kb = stage_col(s, 0);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const int vo = live ? (kb == kb_last ? voff_f_last(k) : voffs_f[k]) : kOutOfRange;
          dma_b128(db, &b_ring[slot0][(8 * wave + 2 * k) * (kPanel * 4)], vo, kb * b_kstride);
        }
        return;
      }
      if (a_wave) {
        const int idx = base + wave;
        const bool live = idx < nt;
        dma_b128(da, &a_ring[slot0 + wave][0], live ? voff_a : kOutOfRange,
                 (begin + (live ? idx : 0)) * (kTile * kTile));
      }
      // A live stage with K % 32 == 0 (no slab crosses K) needs no per-tile
      // offset selects.
      if (base + RT <= nt && kb_last < 0) {
#pragma unroll
        for (int u = 0; u < RT; ++u)
          dma_b128(db, &b_ring[slot0 + u][wave * (kSlotBytes / kWaves)], voffd, stage_col(s, u) * b_kstride);
        return;
      }
#pragma unroll
      for (int u = 0; u < RT; ++u) {
        const int kb = stage_col(s, u);
        const int vo = base + u < nt ? (kb == kb_last ? voffd_last : voffd) : kOutOfRange;
        dma_b128(db, &b_ring[slot0 + u][wave * (kSlotBytes / kWaves)], vo, kb * b_kstride);
      }
    };
#pragma unroll
    for (int s = 0; s < kDmaStages - 1; ++s)
      if (s < ns) issue_stage(s);
    TRACE_POINT(1);
    for (int s = 0; s < ns_loop; ++s) {
      // Past this group's last stage (s >= ns) ahead is negative: wait for all.
      const int ahead = min(ns - 1, s + kDmaStages - 2) - s;  // stages issued after s
      if (kF32 || k16) wait_stages<5>(ahead);
      else if (kBF32 || kF8B16) {
        if (a_wave) wait_stages<5>(ahead);
        else wait_stages<4>(ahead);
      } else if (a_wave) wait_stages<1 + RT>(ahead);
      else wait_stages<RT>(ahead);
      if (s == 0) {
        // The windows were issued before stage 0, so they have landed too.
        colw = win[lane];
        if constexpr (kScales) scw = __int_as_float(win[64 + lane]);
        TRACE_POINT(5);
      }
      // Every wave's part of stage s has landed, and every wave has finished
      // reading stage s - 1, whose slots the next issue overwrites.
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
      if (s + kDmaStages - 1 < ns) {
        // One-ring workgroups (five per CU): the refill is issued at raised
        // wave priority, ahead of the other workgroups' scaled adds on the
        // same SIMD (c5: 86.3-88.5 -> 85.6-87.2 us cold, 98-101 -> 96-97 hot;
        // the two-ring kernel measured slower with it).
        if constexpr (KS == 1) __builtin_amdgcn_s_setprio(3);
        issue_stage(s + kDmaStages - 1);
        if constexpr (KS == 1) __builtin_amdgcn_s_setprio(0);
      }
      if (KS > 1 && s >= ns) continue;  // the other group's extra stage
      const int slot0 = (s % kDmaStages) * kStageTiles;
      const int base = (s * KS + sg) * kStageTiles;
      if constexpr (kF32) {
        // fp32 tile: lane (i, g) holds A row i, columns 16 g .. +15 and B column
        // 32 wave + i (of the panel), rows 16 g .. +15; MFMA s takes k pair
        // (s, 16 + s) from both operands.
        const uint8_t* as = reinterpret_cast<const uint8_t*>(&a_ring[slot0][0]);
        const uint8_t* bs = &b_ring[slot0][0];
        v4f af[4];
#pragma unroll
        for (int q = 0; q < 4; ++q)
          af[q] = *reinterpret_cast<const v4f*>(as + j * (kTile * 4) + (((4 * g + q) ^ (j & 7)) << 4));
        const int colp = wave * kTile + j;
        float bf[16];
#pragma unroll
        for (int s2 = 0; s2 < 16; ++s2)
          bf[s2] = *reinterpret_cast<const float*>(bs + (16 * g + s2) * (kPanel * 4) +
                                                   (((colp >> 2) ^ (g << 3)) << 4) + (colp & 3) * 4);
#pragma unroll
        for (int s2 = 0; s2 < 16; ++s2)
          acc = __builtin_amdgcn_mfma_f32_32x32x2f32(af[s2 >> 2][s2 & 3], bf[s2], acc, 0, 0, 0);
      } else if constexpr (k16) {
        // 16-bit tiles on v_mfma_f32_32x32x16_{bf16,f16}, two per tile: MFMA h
        // takes k = 16 h + 8 g .. + 7 for lane (i, g), A row i (one 16-byte
        // read) and B column 32 wave + i (two ds_read_b64_tr_b16, each giving
        // four k of one column: the 16 lanes of a read fetch a 4-row x
        // 16-column block, 8 bytes each in row-major order, and lane t gets
        // column t).  Tiles past the item's end were loaded as zeros.
        const int i = j & 15;
        typedef short v4h16 __attribute__((ext_vector_type(4)));
        typedef short v8h16 __attribute__((ext_vector_type(8)));
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const uint8_t* as = reinterpret_cast<const uint8_t*>(&a_ring[slot0 + u][0]);
          const uint8_t* bs = &b_ring[slot0 + u][0];
          v4i av[2];
          v8h16 bv[2];
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            av[h] = *reinterpret_cast<const v4i*>(as + j * (kTile * 2) + (((2 * h + g) ^ ((j >> 2) & 3)) << 4));
            v4h16 t[2];
#pragma unroll
            for (int r = 0; r < 2; ++r) {
              const int row = 16 * h + 8 * g + 4 * r + (i >> 2);
              const int gq = 4 * wave + 2 * (j >> 4) + ((i & 3) >> 1);
              const uint8_t* a = bs + row * (kPanel * 2) + ((gq ^ ((row & 3) << 2)) << 4) + 8 * (i & 1);
              t[r] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                  (__attribute__((address_space(3))) v4h16*)(const_cast<uint8_t*>(a)));
            }
            bv[h] = v8h16{t[0][0], t[0][1], t[0][2], t[0][3], t[1][0], t[1][1], t[1][2], t[1][3]};
          }
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            if constexpr (ELT == kEltBf16)
              acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf, av[h]),
                                                            __builtin_bit_cast(v8bf, bv[h]), acc, 0, 0, 0);
            else
              acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8hf, av[h]),
                                                           __builtin_bit_cast(v8hf, bv[h]), acc, 0, 0, 0);
          }
        }
      } else if constexpr (kF8B16) {
        // E4M3 tiles times a 16-bit B: lane (i, g) decodes its 16 codes of A
        // row i (k = 16 g .. + 15) exactly to B's 16-bit type; MFMA h takes
        // k = 16 g + 8 h .. + 7 of A and of B column 32 wave + i (two
        // transposed reads, as for 16-bit tiles).  Each tile's product is
        // scaled into the fp32 accumulators.
        const int i = j & 15;
        typedef short v4h16 __attribute__((ext_vector_type(4)));
        typedef short v8h16 __attribute__((ext_vector_type(8)));
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const v4i araw = a_ring[slot0 + u][lane];
          v4i a8[2];
          {
            uint32_t d[8];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              if constexpr (ELT == kEltFp8Bf16) e4m3x4_to_bf16((uint32_t)araw[q], d[2 * q], d[2 * q + 1]);
              else e4m3x4_to_f16((uint32_t)araw[q], d[2 * q], d[2 * q + 1]);
            }
            a8[0] = v4i{(int)d[0], (int)d[1], (int)d[2], (int)d[3]};
            a8[1] = v4i{(int)d[4], (int)d[5], (int)d[6], (int)d[7]};
          }
          const uint8_t* bs = &b_ring[slot0 + u][0];
          v8h16 bv[2];
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            v4h16 t[2];
#pragma unroll
            for (int r = 0; r < 2; ++r) {
              const int row = 16 * g + 8 * h + 4 * r + (i >> 2);
              const int gq = 4 * wave + 2 * (j >> 4) + ((i & 3) >> 1);
              const uint8_t* a = bs + row * (kPanel * 2) + ((gq ^ ((row & 3) << 2)) << 4) + 8 * (i & 1);
              t[r] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                  (__attribute__((address_space(3))) v4h16*)(const_cast<uint8_t*>(a)));
            }
            bv[h] = v8h16{t[0][0], t[0][1], t[0][2], t[0][3], t[1][0], t[1][1], t[1][2], t[1][3]};
          }
          v16f part = {};
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            if constexpr (ELT == kEltFp8Bf16)
              part = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf, a8[h]),
                                                             __builtin_bit_cast(v8bf, bv[h]), part, 0, 0, 0);
            else
              part = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8hf, a8[h]),
                                                            __builtin_bit_cast(v8hf, bv[h]), part, 0, 0, 0);
          }
          // Tiles past the item's end were loaded as zeros (a zero product).
          const float sc = bcast(scw, min(base + u, kCgMaxTiles - 1));
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[r] = __builtin_fmaf(sc, part[r], acc[r]);
        }
      } else if constexpr (ELT == kEltFp8F32) {
        // E4M3 tile times fp32 B on the bf16 MFMA: lane (i, g) holds A row i,
        // k = 16 g .. 16 g + 15 (its 16 codes, decoded exactly to bf16) and B
        // column 32 wave + i, the same 16 rows, split into bf16 hi + lo.  MFMA
        // h (h = 0, 1) takes k = 16 g + 8 h .. + 7 from both operands, once
        // with hi and once with lo: A (hi + lo) is within 2^-16 of A B per
        // product, and the tile's scale multiplies the fp32 sum.
        const v4i araw = a_ring[slot0][lane];
        v4i a8[2];
        {
          uint32_t d[8];
#pragma unroll
          for (int q = 0; q < 4; ++q) e4m3x4_to_bf16((uint32_t)araw[q], d[2 * q], d[2 * q + 1]);
          a8[0] = v4i{(int)d[0], (int)d[1], (int)d[2], (int)d[3]};
          a8[1] = v4i{(int)d[4], (int)d[5], (int)d[6], (int)d[7]};
        }
        const uint8_t* bs = &b_ring[slot0][0];
        const int colp = wave * kTile + j;
        float bf[16];
#pragma unroll
        for (int s2 = 0; s2 < 16; ++s2)
          bf[s2] = *reinterpret_cast<const float*>(bs + (16 * g + s2) * (kPanel * 4) +
                                                   (((colp >> 2) ^ (g << 3)) << 4) + (colp & 3) * 4);
        v4i bh[2], bl[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            uint32_t hi, lo;
            split_bf16(bf[8 * h + 2 * q], bf[8 * h + 2 * q + 1], hi, lo);
            bh[h][q] = (int)hi;
            bl[h][q] = (int)lo;
          }
        }
        v16f part = {};
#pragma unroll
        for (int h = 0; h < 2; ++h)
          part = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf, a8[h]), __builtin_bit_cast(v8bf, bh[h]),
                                                         part, 0, 0, 0);
#pragma unroll
        for (int h = 0; h < 2; ++h)
          part = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf, a8[h]), __builtin_bit_cast(v8bf, bl[h]),
                                                         part, 0, 0, 0);
        const float sc = bcast(scw, base);
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[r] = __builtin_fmaf(sc, part[r], acc[r]);
      } else {
        // Every stage runs as a full one: all operand reads first, then RT
        // independent products, so that one tile's scaling overlaps the next
        // MFMA.  The slots of tiles past the item's end were loaded out of
        // range, which writes zeros to LDS, so their integer products are
        // zero; the per-block fold also gives them a zero scale.  One code
        // path keeps the accumulators in place: with a separate path for
        // the item's last, partial stage the compiler copied all 16 of them
        // twice per stage (16 v_mov_b64 per 3-tile stage on c5).
        Frag1 f[RT];
#pragma unroll
        for (int u = 0; u < RT; ++u) {
          f[u].a = a_ring[slot0 + u][lane];
          f[u].b = read_tr(&b_ring[slot0 + u][0], wave, j, g);
        }
        if constexpr (kInt) {
#pragma unroll
          for (int u = 0; u < RT; ++u) A::step(acc, f[u], 0.f);
        } else {
          // Products two tiles ahead of their scaled adds: the VALU work of
          // tile u runs while the MFMA of tile u + 2 executes.
          typename A::Part part[RT];
          part[0] = A::prod(f[0]);
          part[1] = A::prod(f[1]);
#pragma unroll
          for (int u = 0; u < RT; ++u) {
            __builtin_amdgcn_sched_barrier(0);
            if (u + 2 < RT) part[u + 2] = A::prod(f[u + 2]);
            // The select on the scale's bits stays in SGPRs (a float select
            // compiled to v_mov + v_cndmask per tile).
            const int si = __builtin_amdgcn_readlane(__float_as_int(scw), min(base + u, kCgMaxTiles - 1));
            A::fold(acc, part[u], __int_as_float(base + u < nt ? si : 0));
          }
        }
      }
    }
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    TRACE_POINT(6);
    if constexpr (KS > 1) {
      // Group 1 hands its accumulators to group 0 through its own (now idle)
      // B area, word r of lane l at (wave * 16 + r) * 64 + l, and leaves.
      int* xb = reinterpret_cast<int*>(&b_lds[kSlots][0]) + wave * 16 * 64;
      if (sg == 1) {
#pragma unroll
        for (int r = 0; r < 16; ++r)  // (__builtin_bit_cast of an element here compiled to element 0 for every r)
          xb[r * 64 + lane] = kInt ? (int)acc[r] : __float_as_int((float)acc[r]);
      }
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
      // On a split row group 1 stays, idle, for the split protocol's two
      // workgroup barriers below and leaves after them.
      if (sg == 1 && split_tile < 0) {
        TRACE_FLUSH();
        return;
      }
      if (sg == 0) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          if constexpr (kInt) acc[r] += xb[r * 64 + lane];
          else acc[r] += __int_as_float(xb[r * 64 + lane]);
        }
      }
    }
  } else if (nt > 0) {
    {
      const int ci = begin + min(lane, nt - 1);
      colw = __builtin_amdgcn_raw_buffer_load_b32(rcol, ci * 4, 0, 0);
      if constexpr (kScales)
        scw = __int_as_float(__builtin_amdgcn_raw_buffer_load_b32(rsc, p.per_tensor_a ? 0 : ci * 4, 0, 0));
    }
    CgBatch X, Y;
    take_cols(0);
    issue(X, 0);
    TRACE_POINT(1);
    int bb = 0;
    // Unrolled by two so that the two batch buffers keep fixed registers;
    // every issued load is unconditional within its branch, which keeps the
    // compiler's vmcnt waits exact.
    while (true) {
      if ((bb + 1) * kCgBatch < nt) {
        take_cols(bb + 1);
        issue(Y, bb + 1);
        consume(X, bb);
        ++bb;
        if ((bb + 1) * kCgBatch < nt) {
          take_cols(bb + 1);
          issue(X, bb + 1);
          consume(Y, bb);
          ++bb;
          continue;
        }
        consume(Y, bb);
        break;
      }
      consume(X, bb);
      break;
    }
  }
  TRACE_POINT(2);

  // MFMA 32x32 result layout: lane (j, g), register r holds row
  // 8 (r / 4) + 4 g + r % 4 of column j.
  if (split_tile >= 0) {
    // Split row: publish this chunk's partial block with agent-coherent (sc1)
    // stores, count arrivals per (row, panel), and let the last chunk read
    // every partial back with agent-coherent loads and reduce them in chunk
    // order, so the result does not depend on timing.
    // Partial blocks: register 4 q + e of lane l at dword (q * 64 + l) * 4 + e
    // of the wave's 4 KB block, so that each 16-byte store or load
    // instruction covers 1 KB contiguously.  sc1 makes them agent-coherent
    // (L2), as relaxed agent-scope atomics would be.
    constexpr int kSc1 = 16;
    const int nchunks = itp->nchunks, slot = itp->slot, chunk = itp->chunk;
    constexpr size_t kBlock = (size_t)kTile * kTile;  // one wave's block
    int* part = static_cast<int*>(p.partials);
    auto block_of = [&](int c) -> const int* {
      return part + (((size_t)(slot + c) * p.n_panels + panel) * kWaves + wave) * kBlock;
    };
    if (sg == 0) {  // (two wave groups: group 0 holds the combined block)
      const Rsrc rp = make_rsrc(block_of(chunk));
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        v4i w;
#pragma unroll
        for (int e = 0; e < 4; ++e) w[e] = kInt ? (int)acc[4 * q + e] : __float_as_int((float)acc[4 * q + e]);
        __builtin_amdgcn_raw_buffer_store_b128(w, rp, (q * 64 + lane) * 16, 0, kSc1);
      }
    }
    publish_wait();  // this wave's partial stores are acknowledged
    __syncthreads();
    unsigned* ctr = p.counters + (size_t)split_tile * p.n_panels + panel;
    if (tid == 0) {
      const unsigned old = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      s_last = (old == (unsigned)(nchunks - 1));
    }
    __syncthreads();
    if (!s_last || sg == 1) {
      TRACE_FLUSH();
      return;
    }
    if (tid == 0) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    compiler_order();  // the partial loads stay below the arrival count
    // Reduce in chunk order (deterministic), with the loads of four chunks
    // in flight at a time.
    typename A::Reg sum = {};
    for (int c0 = 0; c0 < nchunks; c0 += 4) {
      v4i x[4][4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const bool live = c0 + k < nchunks;
        const Rsrc rp = make_rsrc(block_of(live ? c0 + k : c0));
#pragma unroll
        for (int q = 0; q < 4; ++q)
          x[k][q] = __builtin_amdgcn_raw_buffer_load_b128(rp, live ? (q * 64 + lane) * 16 : kOutOfRange, 0, kSc1);
      }
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        if (c0 + k < nchunks) {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int v = x[k][r >> 2][r & 3];
            if constexpr (kInt) sum[r] += v;
            else sum[r] += __int_as_float(v);
          }
        }
      }
    }
    acc = sum;
  }

  float mul = 1.f;
  if constexpr (EPI == VOID_EPI_ROW_MEAN) {
    // int_quant.py:519-526: S = sum fl(s_a * s_b) in tile order over the
    // whole block-row, then S / n.  The row's scales sit one per lane and
    // are folded sequentially with readlane.
    float S = 0.f;
    for (int t0 = rb; t0 < re; t0 += 64) {
      const int n = min(64, re - t0);
      const float mine = t0 == rb ? row_scale
                                  : (p.per_tensor_a ? p.a_scale[0] : p.a_scale[t0 + min(lane, n - 1)]);
      for (int q = 0; q < n; ++q) S = __fadd_rn(S, __fmul_rn(bcast(mine, q), sb));
    }
    mul = (re > rb) ? __fdiv_rn(S, (float)(re - rb)) : 0.f;
  } else if constexpr (EPI == VOID_EPI_PER_BLOCK) {
    mul = kFloat ? 1.f : sb;
  }

  constexpr int esz = (OUT == VOID_DT_F32 || OUT == VOID_DT_I32) ? 4 : 2;
  const Rsrc rc = make_rsrc(p.c);
  const int ldc = (int)p.ldc;
  const int voff_c = ((4 * g) * ldc + col) * esz;
  // Per-row bias (FusedSparseLinear): the bias of output row r.
  auto row_bias = [&](int r) -> float { return p.bias[min(r, p.M - 1)]; };
  const int row0 = row * kTile;
  const bool full = row0 + kTile <= p.M && cg * kTile + kTile <= p.N;
  // LDS-DMA variant, whole block in range and 16-byte aligned rows: the
  // wave's 32 x 32 block goes through its own row-major LDS area (the B ring
  // is idle after the loop's last barrier) and leaves as 16-byte stores,
  // each covering 8 (f32, i32) or 16 (bf16, f16) full 32-column row
  // segments: 4 or 2 store instructions per lane in place of 16.
  if constexpr (DMA) {
    const bool vec = full && ((reinterpret_cast<uintptr_t>(p.c) | (uintptr_t)(ldc * esz)) & 15) == 0;
    if (vec) {
      constexpr int kRowB = kTile * esz + 16;  // padded row stride: the two half waves hit other banks
      uint8_t* stg = &b_lds[0][0] + wave * (kTile * kRowB);
      float xv[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int rr = 8 * (r >> 2) + (r & 3) + 4 * g;
        float x;
        if constexpr (EPI == VOID_EPI_ROW_MEAN || EPI == VOID_EPI_PER_BLOCK) x = __fmul_rn((float)acc[r], mul);
        else x = 0.f;
        if (p.bias) x = __fadd_rn(x, p.bias_per_row ? row_bias(row0 + rr) : bias);
        xv[r] = x;
      }
      if constexpr (OUT != VOID_DT_I32) activate_all(xv, p.activation);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int rr = 8 * (r >> 2) + (r & 3) + 4 * g;
        const float x = xv[r];
        uint8_t* d = stg + rr * kRowB + j * esz;
        if constexpr (OUT == VOID_DT_F32) *reinterpret_cast<float*>(d) = x;
        else if constexpr (OUT == VOID_DT_I32) *reinterpret_cast<int*>(d) = (int)acc[r];
        else *reinterpret_cast<uint16_t*>(d) = (uint16_t)(OUT == VOID_DT_BF16 ? f32_to_bf16_bits(x) : f32_to_f16_bits(x));
      }
      constexpr int kChunks = kTile * esz / 16;  // 16-byte chunks per row segment
      constexpr int kRowsPer = 64 / kChunks;     // rows per store instruction
      const int ch = lane % kChunks;
      TRACE_POINT(3);
#pragma unroll
      for (int k = 0; k < kTile / kRowsPer; ++k) {
        const int rw = k * kRowsPer + lane / kChunks;
        const v4i v = *reinterpret_cast<const v4i*>(stg + rw * kRowB + ch * 16);
        __builtin_amdgcn_raw_buffer_store_b128(v, rc, ((row0 + rw) * ldc + cg * kTile) * esz + ch * 16, 0, kStoreStream);
      }
      TRACE_POINT(4);
      TRACE_FLUSH();
      return;
    }
  }
  // Each store instruction writes one full 32-column row segment per half
  // wave (128 bytes for f32).
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int rr = 8 * (r >> 2) + (r & 3);
    const int soff = (row0 + rr) * ldc * esz;
    float x;
    if constexpr (EPI == VOID_EPI_ROW_MEAN) x = __fmul_rn((float)acc[r], mul);
    else if constexpr (EPI == VOID_EPI_PER_BLOCK) x = __fmul_rn((float)acc[r], mul);
    else x = 0.f;
    if (p.bias) x = __fadd_rn(x, p.bias_per_row ? row_bias(row0 + rr + 4 * g) : bias);
    x = activate(x, p.activation);
    if (full || (row0 + rr + 4 * g < p.M && col < p.N)) {
      if constexpr (OUT == VOID_DT_F32) {
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_int(x), rc, voff_c, soff, 0);
      } else if constexpr (OUT == VOID_DT_I32) {
        __builtin_amdgcn_raw_buffer_store_b32((int)acc[r], rc, voff_c, soff, 0);
      } else {
        const uint32_t h = OUT == VOID_DT_BF16 ? f32_to_bf16_bits(x) : f32_to_f16_bits(x);
        __builtin_amdgcn_raw_buffer_store_b16((unsigned short)h, rc, voff_c, soff, 0);
      }
    }
  }
  TRACE_POINT(4);
  TRACE_FLUSH();
}

template <int ELT, int EPI, int OUT, bool BCOL, bool DMA = false, int RT = kDmaTiles, int KS = 1>
int launch_cg(const Params& p, int grid, hipStream_t stream) {
  const int map_word = p.xcd_exact | p.pair_snake << 1 | p.item_piles << 2 | p.panel_group << 8;
  hipLaunchKernelGGL((spmm_cg_kernel<ELT, EPI, OUT, BCOL, DMA, RT, KS>), dim3(grid), dim3(kThreads * KS), 0, stream,
                     p.items, map_word, p.n_items, p.n_panels, p);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(VOID_ERR_HIP, "kernel launch failed: %s", hipGetErrorString(e));
  return VOID_OK;
}


// B layouts: column-major (direct 16-byte loads), row-major through LDS
// (16-byte aligned rows), row-major with in-register transposes (4-byte
// aligned rows), or bytewise (anything else).
enum Layout { kColVec, kColByte, kRowLds, kRowVec, kRowByte };

// ---------------------------------------------------------------------------
// Float kernel (void_spmm_f32): fp32 tiles times fp32 B, the reference's
// float path (void_spmm, ops.py:148-213, and the activation kernel of
// fusion.py:98-198), on v_mfma_f32_32x32x2_f32: exact fp32 products with
// fp32 accumulation, no quantisation.
//
// One workgroup = 4 waves on one work item x one 128-column panel.  The
// waves take the item's tiles round-robin (wave w: tiles w, w+4, ...) and
// each computes all 128 columns as four 32x32 accumulators; lane (j, g)
// feeds MFMA c with column 4j + c, so one 16-byte load brings it four
// columns' values of one B row.  A tile: lane (j, g) holds row j, k = 16g ..
// 16g+15 (four 16-byte loads); MFMA s (s < 16) takes k = 16g + s from both
// operands, so the k order agrees for A and B.  Per tile and wave: 20 loads
// and 64 MFMAs of 64 cycles -- the kernel is MFMA-bound, so the next tile's
// loads (one tile ahead) hide the memory latency.  Partial sums of the four
// waves meet in LDS, as in spmm_bsr_kernel, and split rows use the same
// coherent fix-up.

struct F32Tile {
  v4f a[4];   // A[j][16g + 4q .. 16g + 4q + 3]
  v4f b[16];  // B[32 kb + 16g + s][col0 .. col0 + 3]
};

template <int OUT, bool VEC>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) void spmm_f32_kernel(Params p) {
  __shared__ __attribute__((aligned(16))) float red[kWaves][kTile][kRedStride];
  int& s_last = *reinterpret_cast<int*>(&red[0][0][kPanel]);  // padding word: split-row arrival flag

  TRACE_DECL;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int j = lane & 31, g = lane >> 5;

  int item_idx, panel;
  if (!wg_map(p, item_idx, panel)) return;
  const void_work_item* itp = p.items + item_idx;
  const int row = itp->row, begin = itp->begin, end = itp->end, split_tile = itp->tile;
  const int nt = end - begin;
  const int col0 = panel * kPanel + j * kColsPerLane;
  TRACE_POINT(0);

  const float* tiles = reinterpret_cast<const float*>(p.tiles);
  const float* B = reinterpret_cast<const float*>(p.b);
  // Block column of tile i (i < 64) in lane i; the host keeps items at <= 64 tiles.
  const int col_64 = nt > 0 ? p.col_idx[begin + min(lane, nt - 1)] : 0;
  const int bcol = col0 < p.N ? col0 : 0;  // past N: any valid column, never stored

  float bias[4] = {0.f, 0.f, 0.f, 0.f};  // per-column bias of this lane's columns
  if (p.bias && !p.bias_per_row) {
#pragma unroll
    for (int c = 0; c < 4; ++c) bias[c] = p.bias[min(col0 + c, p.N - 1)];
  }

  v16f acc[kColsPerLane] = {};
  auto load = [&](F32Tile& x, int idx) {  // idx < nt, wave-uniform
    const int kb = __builtin_amdgcn_readlane(col_64, idx);
    const float* ap = tiles + (int64_t)(begin + idx) * (kTile * kTile) + j * kTile + 16 * g;
#pragma unroll
    for (int q = 0; q < 4; ++q) x.a[q] = *reinterpret_cast<const v4f*>(ap + 4 * q);
#pragma unroll
    for (int s = 0; s < 16; ++s) {
      const int k = min(kb * kTile + 16 * g + s, p.K - 1);  // rows past K meet A's zero padding
      const float* bp = B + (int64_t)k * p.ldb;
      if constexpr (VEC) {
        x.b[s] = *reinterpret_cast<const v4f*>(bp + bcol);
      } else {
        v4f v;
#pragma unroll
        for (int c = 0; c < 4; ++c) v[c] = bp[min(col0 + c, p.N - 1)];
        x.b[s] = v;
      }
    }
  };
  auto consume = [&](const F32Tile& x) {
#pragma unroll
    for (int s = 0; s < 16; ++s) {
      const float a = x.a[s >> 2][s & 3];
#pragma unroll
      for (int c = 0; c < kColsPerLane; ++c)
        acc[c] = __builtin_amdgcn_mfma_f32_32x32x2f32(a, x.b[s][c], acc[c], 0, 0, 0);
    }
  };
  if (wave < nt) {
    // Unrolled by two with fixed buffers; the load of the next tile is
    // unconditional (past the end it re-reads the current one), which keeps
    // the compiler's vmcnt waits exact.
    F32Tile X, Y;
    load(X, wave);
    for (int i = wave;;) {
      load(Y, i + kWaves < nt ? i + kWaves : i);
      consume(X);
      i += kWaves;
      if (i >= nt) break;
      load(X, i + kWaves < nt ? i + kWaves : i);
      consume(Y);
      i += kWaves;
      if (i >= nt) break;
    }
  }
  TRACE_POINT(2);

  // Cross-wave reduction.  MFMA result layout: lane (j, g), register r holds
  // row 8 (r / 4) + 4 g + r % 4; MFMA c holds column 4j + c.
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int rr = 8 * (r >> 2) + 4 * g + (r & 3);
    *reinterpret_cast<v4f*>(&red[wave][rr][red_col(rr, 4 * j)]) = v4f{acc[0][r], acc[1][r], acc[2][r], acc[3][r]};
  }
  __syncthreads();
  v4f sum[kRowsPerWave / 2];
#pragma unroll
  for (int i = 0; i < kRowsPerWave / 2; ++i) {
    const int rr = wave * kRowsPerWave + 2 * i + g;
    v4f s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int w = 0; w < kWaves; ++w) s += *reinterpret_cast<const v4f*>(&red[w][rr][red_col(rr, 4 * j)]);
    sum[i] = s;
  }
  TRACE_POINT(3);

  if (split_tile >= 0) {
    // Split row: the same coherent publish / count / reduce-in-chunk-order
    // protocol as spmm_bsr_kernel.
    const int nchunks = itp->nchunks, slot = itp->slot, chunk = itp->chunk;
    const size_t tile_elems = (size_t)kTile * kPanel;
    int* part = static_cast<int*>(p.partials);
#pragma unroll
    for (int i = 0; i < kRowsPerWave / 2; ++i) {
      const int rr = wave * kRowsPerWave + 2 * i + g;
      const size_t off = ((size_t)(slot + chunk) * p.n_panels + panel) * tile_elems + (size_t)rr * kPanel + 4 * j;
#pragma unroll
      for (int c = 0; c < 4; ++c)
        __hip_atomic_store(part + off + c, __float_as_int(sum[i][c]), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    publish_wait();
    __syncthreads();
    unsigned* ctr = p.counters + (size_t)split_tile * p.n_panels + panel;
    if (tid == 0) {
      const unsigned old = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      s_last = (old == (unsigned)(nchunks - 1));
    }
    __syncthreads();
    if (!s_last) {
      TRACE_FLUSH();
      return;
    }
    if (tid == 0) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    compiler_order();  // the partial loads stay below the arrival count
#pragma unroll
    for (int i = 0; i < kRowsPerWave / 2; ++i) {
      const int rr = wave * kRowsPerWave + 2 * i + g;
      v4f s = {0.f, 0.f, 0.f, 0.f};
      for (int ch = 0; ch < nchunks; ++ch) {
        const size_t off = ((size_t)(slot + ch) * p.n_panels + panel) * tile_elems + (size_t)rr * kPanel + 4 * j;
#pragma unroll
        for (int c = 0; c < 4; ++c)
          s[c] += __int_as_float(__hip_atomic_load(part + off + c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
      }
      sum[i] = s;
    }
  }

#pragma unroll
  for (int i = 0; i < kRowsPerWave / 2; ++i) {
    const int rr = wave * kRowsPerWave + 2 * i + g;
    float v[4];
    int vi[4];
    const int grow = row * kTile + rr;
    const float rbias = (p.bias && p.bias_per_row) ? p.bias[min(grow, p.M - 1)] : 0.f;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      float x = sum[i][c];
      if (p.bias) x = __fadd_rn(x, p.bias_per_row ? rbias : bias[c]);
      v[c] = activate(x, p.activation);
      vi[c] = 0;
    }
    store4<OUT, VEC>(p, grow, col0, v, vi);
  }
  TRACE_POINT(4);
  TRACE_FLUSH();
}

template <int OUT, bool VEC>
int launch_f32(const Params& p, int grid, hipStream_t stream) {
  hipLaunchKernelGGL((spmm_f32_kernel<OUT, VEC>), dim3(grid), dim3(kThreads), 0, stream, p);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(VOID_ERR_HIP, "kernel launch failed: %s", hipGetErrorString(e));
  return VOID_OK;
}

template <int ELT, int EPI, int OUT>
int launch_layout(const Params& p, int grid, hipStream_t s, int layout) {
  switch (layout) {
    case kColVec: return launch<ELT, EPI, OUT, true, true>(p, grid, s);
    case kColByte: return launch<ELT, EPI, OUT, true, false>(p, grid, s);
    case kRowLds: return launch<ELT, EPI, OUT, false, true, true>(p, grid, s);
    case kRowVec: return launch<ELT, EPI, OUT, false, true>(p, grid, s);
    default: return launch<ELT, EPI, OUT, false, false>(p, grid, s);
  }
}

template <int ELT, int EPI>
int launch_out(const Params& p, int grid, hipStream_t s, int layout, int out) {
  switch (out) {
    case VOID_DT_F32: return launch_layout<ELT, EPI, VOID_DT_F32>(p, grid, s, layout);
    case VOID_DT_BF16: return launch_layout<ELT, EPI, VOID_DT_BF16>(p, grid, s, layout);
    case VOID_DT_F16: return launch_layout<ELT, EPI, VOID_DT_F16>(p, grid, s, layout);
    default: return fail(VOID_ERR_UNSUPPORTED, "out_dtype %d not supported with this epilogue", out);
  }
}

size_t counters_bytes(int32_t n_split_tiles, int32_t n_panels) {
  return ((size_t)n_split_tiles * n_panels * sizeof(unsigned) + 255) & ~(size_t)255;
}

int n_panels_for(int32_t N) { return (N + kPanel - 1) / kPanel; }

unsigned long long* g_trace = nullptr;  // set by void_debug_set_trace in instrumented builds

// Ring shape of the 16-bit and fp32-B kernels, as for int8: two rings per
// 8-wave workgroup for one-round grids and split plans below four rounds,
// one ring otherwise.  VOID_AMD_KERNEL=cgdk / cgd force one or the other.
bool two_rings(int32_t n_split_tiles, int64_t grid) {
  const char* fk = getenv("VOID_AMD_KERNEL");
  if (fk && (strcmp(fk, "cgdk") == 0 || strcmp(fk, "cgd") == 0)) return strcmp(fk, "cgdk") == 0;
  return n_split_tiles > 0 ? grid < kDeepGridRounds * 1024 : grid <= kPairGridMax;
}

// Split-row counters and partials at fixed places (the allocation-free entry
// point's scratch) in place of a caller's workspace.
struct FixedScratch {
  unsigned* counters;
  size_t counter_bytes;
  void* partials;
  size_t partial_bytes;
};

int run(int elt, const void_bsr_desc* a, const void_dense_args* d, int32_t epilogue,
        const void_plan* plan, void* workspace, size_t workspace_bytes, hipStream_t stream,
        const FixedScratch* fixed = nullptr) {
  g_err[0] = 0;
  if (!a || !d || !plan) return fail(VOID_ERR_ARG, "null descriptor or plan");
  const void_work_item* items = plan->items;
  const int32_t n_items = plan->n_items, n_split_tiles = plan->n_split_tiles;
  if (a->M < 0 || a->K < 0 || d->N < 0 || a->n_blocks < 0)
    return fail(VOID_ERR_ARG, "negative size (M=%d K=%d N=%d n_blocks=%d)", a->M, a->K, d->N, a->n_blocks);
  if (a->n_block_rows != (a->M + kTile - 1) / kTile)
    return fail(VOID_ERR_ARG, "n_block_rows %d != ceil(M/32) for M=%d", a->n_block_rows, a->M);
  if (a->M == 0 || d->N == 0) return VOID_OK;
  if (!d->c) return fail(VOID_ERR_ARG, "null output pointer");
  if (!items || n_items <= 0) return fail(VOID_ERR_ARG, "empty work list for M=%d", a->M);
  if (!a->row_ptr) return fail(VOID_ERR_ARG, "null row_ptr");
  const bool unscaled = elt == kEltF32 || elt == kEltBf16 || elt == kEltF16;
  if (a->n_blocks > 0 && (!a->tiles || !a->col_idx || (!a->scales && !unscaled) || !d->b))
    return fail(VOID_ERR_ARG, "null tile, column, scale or B pointer");
  if (d->ldc < d->N) return fail(VOID_ERR_ARG, "ldc %lld < N %d", (long long)d->ldc, d->N);
  if (d->b_col_major ? d->ldb < a->K : d->ldb < d->N)
    return fail(VOID_ERR_ARG, "ldb %lld too small", (long long)d->ldb);
  if (epilogue < VOID_EPI_RAW_I32 || epilogue > VOID_EPI_PER_BLOCK)
    return fail(VOID_ERR_ARG, "unknown epilogue %d", epilogue);
  if ((epilogue == VOID_EPI_RAW_I32) != (d->out_dtype == VOID_DT_I32))
    return fail(VOID_ERR_UNSUPPORTED, "RAW_I32 epilogue and I32 output go together");
  if (elt == kEltFp8 && epilogue != VOID_EPI_PER_BLOCK)
    return fail(VOID_ERR_UNSUPPORTED, "fp8 SpMM supports only the per-block epilogue");
  const bool b_f32 = elt == kEltF32 || elt == kEltFp8F32;
  if (b_f32 && d->b_col_major) return fail(VOID_ERR_UNSUPPORTED, "an fp32 B must be row-major");
  if (d->bias_per_row && !unscaled)
    return fail(VOID_ERR_UNSUPPORTED, "a per-row bias is supported by the float SpMM only");
  if (b_f32 && plan->chunk_tiles > 64)
    return fail(VOID_ERR_ARG, "an fp32 B takes work items of at most 64 tiles (chunk_tiles %d)", plan->chunk_tiles);
  if (d->activation < VOID_ACT_NONE || d->activation > VOID_ACT_SILU)
    return fail(VOID_ERR_ARG, "unknown activation %d", d->activation);

  const int n_panels = n_panels_for(d->N);
  const int64_t grid64 = (int64_t)n_items * n_panels;
  if (grid64 > 0x7fffffff) return fail(VOID_ERR_ARG, "grid too large");

  Params p{};
  p.tiles = static_cast<const uint8_t*>(a->tiles);
  p.a_scale = a->scales;
  p.row_ptr = a->row_ptr;
  p.col_idx = a->col_idx;
  p.per_tensor_a = a->per_tensor_a;
  p.b = static_cast<const uint8_t*>(d->b);
  p.ldb = d->ldb;
  p.b_scale = d->b_scale;
  p.b_scale_vec = d->b_scale_vec;
  p.bias = d->bias;
  p.c = d->c;
  p.ldc = d->ldc;
  p.M = a->M;
  p.N = d->N;
  p.K = a->K;
  p.n_panels = n_panels;
  p.activation = d->activation;
  p.n_items = n_items;
  p.panel_group = n_panels >= 16 ? n_panels / 8 : 1;
  // With split rows (a long-tailed distribution) every XCD that shares a
  // panel group gets a dealt share of the longest-first list; otherwise the
  // first of them would take all the longest rows.  Without splits the
  // lengths are close and the plain order measured faster.
  int64_t grid_exact = 0;
  {
    const int n_groups = (n_panels + p.panel_group - 1) / p.panel_group;
    p.item_piles = n_split_tiles > 0 ? std::max(1, 8 / n_groups) : 1;
    // One-round unsplit grids (every workgroup resident from the start) take
    // the same dealt layout, with the second half of each XCD's share in
    // reverse: a CU's two workgroups are then one long and one short row.
    if (n_split_tiles == 0 && grid64 <= kPairGridMax) {
      p.item_piles = std::max(1, 8 / n_groups);
      p.pair_snake = 1;
    }
    if ((n_split_tiles > 0 || p.pair_snake) && n_panels % p.panel_group == 0 && 8 % n_groups == 0) {
      p.xcd_exact = 1;
      grid_exact = 8 * (((int64_t)n_items + p.item_piles - 1) / p.item_piles) * p.panel_group;
    }
  }
  p.bias_per_row = d->bias_per_row;
  p.items = items;
  p.trace = g_trace;
  if (n_split_tiles > 0 && fixed) {
    const size_t need_c = counters_bytes(n_split_tiles, n_panels);
    const size_t need_p = void_workspace_bytes(n_split_tiles, plan->n_slots, d->N) - need_c;
    if (need_c > fixed->counter_bytes || need_p > fixed->partial_bytes)
      return fail(VOID_ERR_WORKSPACE,
                  "plan needs %zu bytes of split-row counters and %zu of partials; the allocation-free "
                  "entry point holds at most %zu and %zu (use void_spmm_int8 with a workspace)",
                  need_c, need_p, fixed->counter_bytes, fixed->partial_bytes);
    p.counters = fixed->counters;
    p.partials = fixed->partials;
  } else if (n_split_tiles > 0) {
    if (!workspace) return fail(VOID_ERR_WORKSPACE, "plan splits rows but workspace is null");
    const size_t need = void_workspace_bytes(n_split_tiles, plan->n_slots, d->N);
    if (workspace_bytes < need)
      return fail(VOID_ERR_WORKSPACE, "workspace of %zu bytes, plan needs %zu", workspace_bytes, need);
    p.counters = static_cast<unsigned*>(workspace);
    p.partials = static_cast<char*>(workspace) + counters_bytes(n_split_tiles, n_panels);
  }

  const uintptr_t bu = (uintptr_t)d->b, cu = (uintptr_t)d->c;
  const bool c_ok = (cu % 16 == 0) && (d->ldc % 4 == 0) && (d->N % 4 == 0);
  int layout;
  if (d->b_col_major)
    layout = (c_ok && (bu % 16 == 0) && (d->ldb % 16 == 0) && (a->K % kTile == 0)) ? kColVec : kColByte;
  else if (c_ok && (bu % 16 == 0) && (d->ldb % 16 == 0) && (d->N % 16 == 0))
    layout = kRowLds;
  else
    layout = (c_ok && (bu % 4 == 0) && (d->ldb % 4 == 0)) ? kRowVec : kRowByte;
  if (grid_exact > 0x7fffffff) return fail(VOID_ERR_ARG, "grid too large");
  const int grid = p.xcd_exact ? (int)grid_exact : (int)grid64;

  if (elt == kEltFp8F32) {
    // E4M3 tiles times fp32 B: the LDS-DMA ring only (16-byte aligned rows,
    // N % 4 == 0, 31-bit byte offsets); the Python wrapper pads other shapes.
    const int64_t lim = (int64_t)1 << 31;
    const int esz = (d->out_dtype == VOID_DT_BF16 || d->out_dtype == VOID_DT_F16) ? 2 : 4;
    if (!(c_ok && (bu % 16 == 0) && (d->ldb % 4 == 0)))
      return fail(VOID_ERR_UNSUPPORTED, "E4M3 x fp32 SpMM needs 16-byte aligned B and C rows and N %% 4 == 0");
    if (!((int64_t)a->n_blocks * kTile * kTile < lim && (int64_t)((a->K + kTile - 1) / kTile) * kTile * d->ldb * 4 < lim &&
          (int64_t)a->M * d->ldc * esz < lim))
      return fail(VOID_ERR_UNSUPPORTED, "E4M3 x fp32 SpMM operands must stay below 2 GiB");
    const bool pair = two_rings(n_split_tiles, grid);
    switch (d->out_dtype) {
      case VOID_DT_F32:
        return pair ? launch_cg<kEltFp8F32, VOID_EPI_PER_BLOCK, VOID_DT_F32, false, true, kDmaTiles, 2>(p, grid, stream)
                    : launch_cg<kEltFp8F32, VOID_EPI_PER_BLOCK, VOID_DT_F32, false, true>(p, grid, stream);
      case VOID_DT_BF16:
        return pair ? launch_cg<kEltFp8F32, VOID_EPI_PER_BLOCK, VOID_DT_BF16, false, true, kDmaTiles, 2>(p, grid, stream)
                    : launch_cg<kEltFp8F32, VOID_EPI_PER_BLOCK, VOID_DT_BF16, false, true>(p, grid, stream);
      case VOID_DT_F16:
        return pair ? launch_cg<kEltFp8F32, VOID_EPI_PER_BLOCK, VOID_DT_F16, false, true, kDmaTiles, 2>(p, grid, stream)
                    : launch_cg<kEltFp8F32, VOID_EPI_PER_BLOCK, VOID_DT_F16, false, true>(p, grid, stream);
      default: return fail(VOID_ERR_UNSUPPORTED, "E4M3 x fp32 SpMM writes f32, bf16 or f16");
    }
  }
  if (elt == kEltBf16 || elt == kEltF16 || elt == kEltFp8Bf16 || elt == kEltFp8F16) {
    // A 16-bit B (with 16-bit or E4M3 tiles): the LDS-DMA ring only
    // (row-major B and C with 16-byte aligned rows, N % 8 == 0, items of at
    // most 64 tiles, 31-bit byte offsets).  The Python wrappers take the
    // fp32 B kernels otherwise.
    const int64_t lim = (int64_t)1 << 31;
    const int64_t a_tile_bytes = (elt == kEltBf16 || elt == kEltF16) ? 2048 : 1024;
    const int esz = (d->out_dtype == VOID_DT_BF16 || d->out_dtype == VOID_DT_F16) ? 2 : 4;
    if (d->b_col_major || !(c_ok && (bu % 16 == 0) && (d->ldb % 8 == 0) && (d->N % 8 == 0)))
      return fail(VOID_ERR_UNSUPPORTED, "16-bit SpMM needs a row-major B, 16-byte aligned B and C rows and N %% 8 == 0");
    if (plan->chunk_tiles > kCgMaxTiles)
      return fail(VOID_ERR_ARG, "16-bit SpMM takes work items of at most %d tiles (chunk_tiles %d)", kCgMaxTiles,
                  plan->chunk_tiles);
    if (!((int64_t)a->n_blocks * a_tile_bytes < lim && (int64_t)((a->K + kTile - 1) / kTile) * kTile * d->ldb * 2 < lim &&
          (int64_t)a->M * d->ldc * esz < lim))
      return fail(VOID_ERR_UNSUPPORTED, "16-bit SpMM operands must stay below 2 GiB");
    const bool pair = two_rings(n_split_tiles, grid);
    auto go16 = [&](auto elt_c) -> int {
      constexpr int E = decltype(elt_c)::value;
      auto pick = [&](auto out_c) -> int {
        constexpr int O = decltype(out_c)::value;
        if (pair) return launch_cg<E, VOID_EPI_PER_BLOCK, O, false, true, kDmaTiles, 2>(p, grid, stream);
        return launch_cg<E, VOID_EPI_PER_BLOCK, O, false, true>(p, grid, stream);
      };
      switch (d->out_dtype) {
        case VOID_DT_F32: return pick(std::integral_constant<int, VOID_DT_F32>{});
        case VOID_DT_BF16: return pick(std::integral_constant<int, VOID_DT_BF16>{});
        case VOID_DT_F16: return pick(std::integral_constant<int, VOID_DT_F16>{});
        default: return fail(VOID_ERR_UNSUPPORTED, "16-bit SpMM writes f32, bf16 or f16");
      }
    };
    switch (elt) {
      case kEltBf16: return go16(std::integral_constant<int, kEltBf16>{});
      case kEltF16: return go16(std::integral_constant<int, kEltF16>{});
      case kEltFp8Bf16: return go16(std::integral_constant<int, kEltFp8Bf16>{});
      default: return go16(std::integral_constant<int, kEltFp8F16>{});
    }
  }
  if (elt == kEltF32) {
    const bool vec = c_ok && (bu % 16 == 0) && (d->ldb % 4 == 0) && (d->N % 4 == 0);
    // The column-group LDS-DMA ring for row-major B with 16-byte aligned rows,
    // items of at most 64 tiles and 31-bit byte offsets; VOID_AMD_KERNEL=f32
    // keeps the fp32 kernel of its own (the fallback for everything else).
    const char* fk = getenv("VOID_AMD_KERNEL");
    const int64_t lim = (int64_t)1 << 31;
    const bool ring_ok = vec && !d->b_col_major && plan->chunk_tiles <= kCgMaxTiles &&
                         (int64_t)a->n_blocks * kTile * kTile * 4 < lim &&
                         (int64_t)((a->K + kTile - 1) / kTile) * kTile * d->ldb * 4 < lim &&
                         (int64_t)a->M * d->ldc * 4 < lim && !(fk && strcmp(fk, "f32") == 0);
    if (ring_ok) {
      const bool pair = two_rings(n_split_tiles, grid);
      switch (d->out_dtype) {
        case VOID_DT_F32:
          return pair ? launch_cg<kEltF32, VOID_EPI_PER_BLOCK, VOID_DT_F32, false, true, kDmaTiles, 2>(p, grid, stream)
                      : launch_cg<kEltF32, VOID_EPI_PER_BLOCK, VOID_DT_F32, false, true>(p, grid, stream);
        case VOID_DT_BF16:
          return pair ? launch_cg<kEltF32, VOID_EPI_PER_BLOCK, VOID_DT_BF16, false, true, kDmaTiles, 2>(p, grid, stream)
                      : launch_cg<kEltF32, VOID_EPI_PER_BLOCK, VOID_DT_BF16, false, true>(p, grid, stream);
        case VOID_DT_F16:
          return pair ? launch_cg<kEltF32, VOID_EPI_PER_BLOCK, VOID_DT_F16, false, true, kDmaTiles, 2>(p, grid, stream)
                      : launch_cg<kEltF32, VOID_EPI_PER_BLOCK, VOID_DT_F16, false, true>(p, grid, stream);
        default: return fail(VOID_ERR_UNSUPPORTED, "float SpMM writes f32, bf16 or f16");
      }
    }
    switch (d->out_dtype) {
      case VOID_DT_F32: return vec ? launch_f32<VOID_DT_F32, true>(p, grid, stream) : launch_f32<VOID_DT_F32, false>(p, grid, stream);
      case VOID_DT_BF16: return vec ? launch_f32<VOID_DT_BF16, true>(p, grid, stream) : launch_f32<VOID_DT_BF16, false>(p, grid, stream);
      case VOID_DT_F16: return vec ? launch_f32<VOID_DT_F16, true>(p, grid, stream) : launch_f32<VOID_DT_F16, false>(p, grid, stream);
      default: return fail(VOID_ERR_UNSUPPORTED, "float SpMM writes f32, bf16 or f16");
    }
  }

  // The column-group kernel addresses every operand with
  // 31-bit buffer offsets; larger operands and the other B layouts use
  // spmm_bsr_kernel.  VOID_AMD_KERNEL=bsr / cg / cgd forces a kernel
  // where it applies (for comparisons and tests; cg is the register-staged
  // column-group loop, cgd its LDS-DMA ring, the default).
  const int esz = (d->out_dtype == VOID_DT_BF16 || d->out_dtype == VOID_DT_F16) ? 2 : 4;
  const int64_t kLim = (int64_t)1 << 31;
  const int64_t b_span = d->b_col_major ? (int64_t)d->N * d->ldb
                                        : (int64_t)((a->K + kTile - 1) / kTile) * kTile * d->ldb;
  const char* force = getenv("VOID_AMD_KERNEL");
  const bool force_bsr = force && strcmp(force, "bsr") == 0;
  const bool force_cg = force && strcmp(force, "cg") == 0;
  const bool force_deep = force && strcmp(force, "cgd3") == 0;
  const bool force_pair = force && strcmp(force, "cgdk") == 0;
  const bool offsets_ok = (int64_t)a->n_blocks * kTile * kTile < kLim && b_span < kLim &&
                          (int64_t)a->M * d->ldc * esz < kLim;

  const bool cg_ok = (layout == kRowLds || layout == kColVec) && plan->chunk_tiles <= kCgMaxTiles && offsets_ok &&
                     !force_bsr;
  if (cg_ok) {
    const bool bcol = layout == kColVec;
    // Row-major B takes the LDS-DMA ring unless VOID_AMD_KERNEL=cg asks for
    // the register-staged loop.
    const bool dma = !bcol && !force_cg;
    // Deep grids (several resident rounds) take the 3-tile ring; VOID_AMD_KERNEL=cgd3
    // forces it.
    // Default ring shapes (measured on c2-c5 and on mid-size uniform grids):
    //  - grids that fit in one round of two 8-wave workgroups per CU (512),
    //    and plans with split rows below four resident rounds: two rings per
    //    workgroup (KS = 2), each wave group running half of the item's
    //    stages, which halves the longest item's chain of stage round trips;
    //  - other grids: the 3-tile ring at five workgroups per CU, whose extra
    //    workgroup hides more of the others' starts and epilogues.
    // VOID_AMD_KERNEL=cgd / cgd3 / cgdk force the 4-tile ring, the 3-tile
    // ring or the two-ring workgroups.
    const bool split_deep = n_split_tiles > 0 && grid >= kDeepGridRounds * 1024;
    const bool pair = force_pair || (!force && (n_split_tiles > 0 ? !split_deep : grid <= kPairGridMax));
    const bool deep = !pair && (force_deep || (!force && (n_split_tiles == 0 || split_deep)));
    auto go = [&](auto elt_c, auto epi_c) -> int {
      constexpr int E = decltype(elt_c)::value, P = decltype(epi_c)::value;
      auto pick = [&](auto out_c) -> int {
        constexpr int O = decltype(out_c)::value;
        if (bcol) return launch_cg<E, P, O, true>(p, grid, stream);
        if (!dma) return launch_cg<E, P, O, false>(p, grid, stream);
        if (deep) return launch_cg<E, P, O, false, true, kDmaTilesDeep>(p, grid, stream);
        if (pair) return launch_cg<E, P, O, false, true, kDmaTiles, 2>(p, grid, stream);
        return launch_cg<E, P, O, false, true>(p, grid, stream);
      };
      if constexpr (P == VOID_EPI_RAW_I32) {
        return pick(std::integral_constant<int, VOID_DT_I32>{});
      } else {
        switch (d->out_dtype) {
          case VOID_DT_F32: return pick(std::integral_constant<int, VOID_DT_F32>{});
          case VOID_DT_BF16: return pick(std::integral_constant<int, VOID_DT_BF16>{});
          case VOID_DT_F16: return pick(std::integral_constant<int, VOID_DT_F16>{});
          default:
            return fail(VOID_ERR_UNSUPPORTED, "out_dtype %d not supported with this epilogue", d->out_dtype);
        }
      }
    };
    using I8 = std::integral_constant<int, kEltI8>;
    using F8 = std::integral_constant<int, kEltFp8>;
    if (elt == kEltFp8) return go(F8{}, std::integral_constant<int, VOID_EPI_PER_BLOCK>{});
    switch (epilogue) {
      case VOID_EPI_RAW_I32: return go(I8{}, std::integral_constant<int, VOID_EPI_RAW_I32>{});
      case VOID_EPI_ROW_MEAN: return go(I8{}, std::integral_constant<int, VOID_EPI_ROW_MEAN>{});
      default: return go(I8{}, std::integral_constant<int, VOID_EPI_PER_BLOCK>{});
    }
  }

  if (elt == kEltI8) {
    switch (epilogue) {
      case VOID_EPI_RAW_I32:
        switch (layout) {
          case kColVec: return launch<kEltI8, VOID_EPI_RAW_I32, VOID_DT_I32, true, true>(p, grid, stream);
          case kColByte: return launch<kEltI8, VOID_EPI_RAW_I32, VOID_DT_I32, true, false>(p, grid, stream);
          case kRowLds: return launch<kEltI8, VOID_EPI_RAW_I32, VOID_DT_I32, false, true, true>(p, grid, stream);
          case kRowVec: return launch<kEltI8, VOID_EPI_RAW_I32, VOID_DT_I32, false, true>(p, grid, stream);
          default: return launch<kEltI8, VOID_EPI_RAW_I32, VOID_DT_I32, false, false>(p, grid, stream);
        }
      case VOID_EPI_ROW_MEAN:
        return launch_out<kEltI8, VOID_EPI_ROW_MEAN>(p, grid, stream, layout, d->out_dtype);
      default:
        return launch_out<kEltI8, VOID_EPI_PER_BLOCK>(p, grid, stream, layout, d->out_dtype);
    }
  }
  return launch_out<kEltFp8, VOID_EPI_PER_BLOCK>(p, grid, stream, layout, d->out_dtype);
}

// ---- Scratch of the allocation-free entry point ---------------------------
//
// The split-row counters and partial blocks of void_spmm_int8_noalloc live in
// this array, which every GPU the library runs on holds from module load to
// process end.  Counters take the first kScratchCounterBytes (up to 262144
// split (tile, panel) pairs), partials the rest, so a plan's partials never
// overlap another plan's counters.  The split-row protocol leaves every
// counter it used at zero, so the region is cleared once per device, at set-up.
// In host code `scratch` is a host-side stand-in, not the device address;
// only the pointer from hipGetSymbolAddress (g_scratch_ptr) is used.
constexpr size_t kScratchBytes = (size_t)32 << 20;
constexpr size_t kScratchCounterBytes = (size_t)1 << 20;
static_assert(kScratchCounterBytes == VOID_NOALLOC_COUNTER_BYTES &&
                  kScratchBytes - kScratchCounterBytes == VOID_NOALLOC_PARTIAL_BYTES,
              "limits stated in void_amd.h");
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

__global__ __launch_bounds__(256) void zero_words_kernel(unsigned* p, int n) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < n) p[i] = 0u;
}

// The scratch address on the current device, looked up (and its counter
// region cleared, on `stream`) at the first call on that device.
int scratch_for_current_device(hipStream_t stream, void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(VOID_ERR_HIP, "hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return fail(VOID_ERR_HIP, "device %d beyond the scratch table", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr)
      return fail(VOID_ERR_HIP, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
    // A fill kernel, not hipMemsetAsync, so that set-up under graph capture
    // records a kernel node.
    const int words = (int)(kScratchCounterBytes / sizeof(unsigned));
    hipLaunchKernelGGL(zero_words_kernel, dim3((words + 255) / 256), dim3(256), 0, stream,
                       static_cast<unsigned*>(ptr), words);
    e = hipGetLastError();
    if (e != hipSuccess) return fail(VOID_ERR_HIP, "scratch clear: %s", hipGetErrorString(e));
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return VOID_OK;
}

}  // namespace

extern "C" {

int void_abi_version(void) { return VOID_AMD_ABI_VERSION; }

const char* void_last_error(void) { return g_err; }

int void_panel_width(void) { return kPanel; }

int void_stream_capture_id(hipStream_t stream, unsigned long long* id) {
  g_err[0] = 0;
  if (!id) return fail(VOID_ERR_ARG, "null id");
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  unsigned long long cid = 0;
  const hipError_t e = hipStreamGetCaptureInfo(stream, &st, &cid);
  if (e != hipSuccess) return fail(VOID_ERR_HIP, "hipStreamGetCaptureInfo: %s", hipGetErrorString(e));
  *id = st == hipStreamCaptureStatusActive ? cid : 0;
  return VOID_OK;
}

int void_device_info(int32_t* compute_units, int32_t* sclk_khz, int32_t* mclk_khz, int32_t* bus_bits) {
  g_err[0] = 0;
  if (!compute_units || !sclk_khz || !mclk_khz || !bus_bits) return fail(VOID_ERR_ARG, "null output pointer");
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  int v[4] = {0, 0, 0, 0};
  const hipDeviceAttribute_t attrs[4] = {hipDeviceAttributeMultiprocessorCount, hipDeviceAttributeClockRate,
                                         hipDeviceAttributeMemoryClockRate, hipDeviceAttributeMemoryBusWidth};
  for (int i = 0; i < 4 && e == hipSuccess; ++i) e = hipDeviceGetAttribute(&v[i], attrs[i], dev);
  if (e != hipSuccess) return fail(VOID_ERR_HIP, "device attributes: %s", hipGetErrorString(e));
  *compute_units = v[0];
  *sclk_khz = v[1];
  *mclk_khz = v[2];
  *bus_bits = v[3];
  return VOID_OK;
}

#ifdef VOID_TRACE
// Instrumented builds only: every launch records 8 realtime stamps per
// workgroup into buf (device memory, >= 8 * grid entries).
void void_debug_set_trace(unsigned long long* buf) { g_trace = buf; }
#endif

int void_streamk_plan(const int32_t* row_ptr, const int32_t* col_idx, int32_t n_block_rows,
                      int32_t chunk_tiles, void_work_item* items, int32_t capacity,
                      int32_t* n_items, int32_t* n_split_tiles, int32_t* n_slots) {
  g_err[0] = 0;
  if (!row_ptr || !n_items || !n_split_tiles || !n_slots || n_block_rows < 0 || chunk_tiles < 1)
    return fail(VOID_ERR_ARG, "bad planner arguments");
  std::vector<void_work_item> out;
  out.reserve(n_block_rows);
  int32_t tiles = 0, slots = 0;
  auto make = [&](int32_t r, int32_t b, int32_t e, int32_t tile, int32_t nch, int32_t ch, int32_t slot) {
    void_work_item w;
    w.row = r;
    w.begin = b;
    w.end = e;
    w.tile = tile;
    w.nchunks = nch;
    w.chunk = ch;
    w.slot = slot;
    w.reserved = 0;
    for (int i = 0; i < VOID_ITEM_INLINE_COLS; ++i) w.cols[i] = (col_idx && b + i < e) ? col_idx[b + i] : -1;
    out.push_back(w);
  };
  for (int32_t r = 0; r < n_block_rows; ++r) {
    const int32_t b = row_ptr[r], e = row_ptr[r + 1];
    if (e < b) return fail(VOID_ERR_ARG, "row_ptr decreases at row %d", r);
    const int32_t n = e - b;
    if (n <= chunk_tiles) {
      make(r, b, e, -1, 1, 0, 0);
      continue;
    }
    const int32_t nch = (n + chunk_tiles - 1) / chunk_tiles;
    for (int32_t c = 0; c < nch; ++c) {
      const int32_t cb = b + (int32_t)((int64_t)c * n / nch);
      const int32_t ce = b + (int32_t)((int64_t)(c + 1) * n / nch);
      make(r, cb, ce, tiles, nch, c, slots);
    }
    tiles += 1;
    slots += nch;
  }
  // Longest items first so that the tail of the dispatch is short ones.  The
  // kernels deal this list among the XCDs that share a panel group when rows
  // were split (wg_tile), so each XCD's share is a balanced mix.
  std::stable_sort(out.begin(), out.end(), [](const void_work_item& x, const void_work_item& y) {
    return (x.end - x.begin) > (y.end - y.begin);
  });
  *n_items = (int32_t)out.size();
  *n_split_tiles = tiles;
  *n_slots = slots;
  if (!items || capacity < (int32_t)out.size())
    return fail(VOID_ERR_CAPACITY, "planner needs %zu items, capacity %d", out.size(), capacity);
  std::memcpy(items, out.data(), out.size() * sizeof(void_work_item));
  return VOID_OK;
}


size_t void_workspace_bytes(int32_t n_split_tiles, int32_t n_slots, int32_t N) {
  if (n_split_tiles <= 0 || N <= 0) return 0;
  const int n_panels = n_panels_for(N);
  return counters_bytes(n_split_tiles, n_panels) + (size_t)n_slots * n_panels * kTile * kPanel * 4;
}

int void_spmm_int8(const void_bsr_desc* a, const void_dense_args* d, int32_t epilogue,
                   const void_plan* plan, void* workspace, size_t workspace_bytes,
                   hipStream_t stream) {
  return run(kEltI8, a, d, epilogue, plan, workspace, workspace_bytes, stream);
}

int void_spmm_int8_noalloc(const void_bsr_desc* a, const void_dense_args* d, int32_t epilogue,
                           const void_plan* plan, hipStream_t stream) {
  g_err[0] = 0;
  if (!plan) return fail(VOID_ERR_ARG, "null plan");
  FixedScratch fs{};
  if (plan->n_split_tiles > 0) {
    void* base = nullptr;
    const int rc = scratch_for_current_device(stream, &base);
    if (rc != VOID_OK) return rc;
    fs.counters = static_cast<unsigned*>(base);
    fs.counter_bytes = kScratchCounterBytes;
    fs.partials = static_cast<char*>(base) + kScratchCounterBytes;
    fs.partial_bytes = kScratchBytes - kScratchCounterBytes;
  }
  return run(kEltI8, a, d, epilogue, plan, nullptr, 0, stream, &fs);
}

int void_spmm_fp8(const void_bsr_desc* a, const void_dense_args* d, const void_plan* plan,
                  void* workspace, size_t workspace_bytes, hipStream_t stream) {
  return run(kEltFp8, a, d, VOID_EPI_PER_BLOCK, plan, workspace, workspace_bytes, stream);
}

int void_spmm_fp8_f32b(const void_bsr_desc* a, const void_dense_args* d, const void_plan* plan,
                       void* workspace, size_t workspace_bytes, hipStream_t stream) {
  if (d && d->out_dtype == VOID_DT_I32) return fail(VOID_ERR_UNSUPPORTED, "E4M3 x fp32 SpMM writes f32, bf16 or f16");
  return run(kEltFp8F32, a, d, VOID_EPI_PER_BLOCK, plan, workspace, workspace_bytes, stream);
}

int void_spmm_f32(const void_bsr_desc* a, const void_dense_args* d, const void_plan* plan,
                  void* workspace, size_t workspace_bytes, hipStream_t stream) {
  if (d && d->out_dtype == VOID_DT_I32) return fail(VOID_ERR_UNSUPPORTED, "float SpMM writes f32, bf16 or f16");
  return run(kEltF32, a, d, VOID_EPI_PER_BLOCK, plan, workspace, workspace_bytes, stream);
}

int void_spmm_fp8_b16(const void_bsr_desc* a, const void_dense_args* d, int32_t b_dtype, const void_plan* plan,
                      void* workspace, size_t workspace_bytes, hipStream_t stream) {
  if (d && d->out_dtype == VOID_DT_I32) return fail(VOID_ERR_UNSUPPORTED, "E4M3 x 16-bit SpMM writes f32, bf16 or f16");
  if (b_dtype != VOID_DT_BF16 && b_dtype != VOID_DT_F16)
    return fail(VOID_ERR_ARG, "b_dtype must be VOID_DT_BF16 or VOID_DT_F16, got %d", b_dtype);
  return run(b_dtype == VOID_DT_BF16 ? kEltFp8Bf16 : kEltFp8F16, a, d, VOID_EPI_PER_BLOCK, plan, workspace,
             workspace_bytes, stream);
}

int void_spmm_bf16(const void_bsr_desc* a, const void_dense_args* d, const void_plan* plan,
                   void* workspace, size_t workspace_bytes, hipStream_t stream) {
  if (d && d->out_dtype == VOID_DT_I32) return fail(VOID_ERR_UNSUPPORTED, "16-bit SpMM writes f32, bf16 or f16");
  return run(kEltBf16, a, d, VOID_EPI_PER_BLOCK, plan, workspace, workspace_bytes, stream);
}

int void_spmm_f16(const void_bsr_desc* a, const void_dense_args* d, const void_plan* plan,
                  void* workspace, size_t workspace_bytes, hipStream_t stream) {
  if (d && d->out_dtype == VOID_DT_I32) return fail(VOID_ERR_UNSUPPORTED, "16-bit SpMM writes f32, bf16 or f16");
  return run(kEltF16, a, d, VOID_EPI_PER_BLOCK, plan, workspace, workspace_bytes, stream);
}

}  // extern "C"
