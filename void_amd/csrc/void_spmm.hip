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
//
// Cross-wave reduction goes through LDS (4 x 16 KB).  Rows that the planner
// split into several items write partial tiles to a workspace; the last
// chunk to arrive (agent-scope atomic counter) sums the partials in chunk
// order and applies the epilogue, so results do not depend on timing.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <vector>

#include "void_amd.h"

extern "C" size_t void_workspace_bytes(int32_t n_split_tiles, int32_t n_slots, int32_t N);

namespace {

constexpr int kTile = 32;
constexpr int kWaves = 4;
constexpr int kColsPerLane = 4;
constexpr int kPanel = 32 * kColsPerLane;  // 128 output columns per workgroup
constexpr int kThreads = 64 * kWaves;

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));

enum Elt { kEltI8 = 0, kEltFp8 = 1 };

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
  int64_t ldb;
  int64_t ldc;
  float b_scale;
  int32_t per_tensor_a;
  int32_t M, N, K;
  int32_t n_panels;
  int32_t activation;
};

// Workgroups are dispatched round-robin over the 8 XCDs.  Remap so that the
// panels of one work item (consecutive logical ids) run on the same XCD and
// share its L2 for the item's A tiles.
__device__ __forceinline__ int xcd_remap(int h, int G) {
  const int per = G >> 3, rem = G & 7;
  const int x = h & 7, s = h >> 3;
  return x < rem ? x * (per + 1) + s : rem * (per + 1) + (x - rem) * per + s;
}

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

// Operand registers of one tile for one lane.
struct Frag {
  v4i a;
  v4i b[kColsPerLane];  // b[c]: 16 k-contiguous bytes of column col0 + c
};

template <bool BCOL, bool VEC>
__device__ __forceinline__ void load_frag(const Params& p, int t, int j, int g, int col0, Frag& f) {
  f.a = *reinterpret_cast<const v4i*>(p.tiles + (size_t)t * (kTile * kTile) + j * kTile + g * 16);
  const int kb = p.col_idx[t];
  const int k0 = kb * kTile + g * 16;
  const int krem = p.K - k0;  // rows of B that exist from k0 on
  if constexpr (!BCOL) {
    const uint8_t* bp = p.b + (int64_t)k0 * p.ldb + col0;
    uint32_t r[16];
    if constexpr (VEC) {
      const bool colok = col0 < p.N;
#pragma unroll
      for (int i = 0; i < 16; ++i)
        r[i] = (colok && i < krem) ? *reinterpret_cast<const uint32_t*>(bp + i * p.ldb) : 0u;
    } else {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        uint32_t w = 0;
#pragma unroll
        for (int c = 0; c < 4; ++c)
          if (i < krem && col0 + c < p.N) w |= (uint32_t)bp[i * p.ldb + c] << (8 * c);
        r[i] = w;
      }
    }
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
    for (int c = 0; c < kColsPerLane; ++c) {
      const uint8_t* bp = p.b + (int64_t)(col0 + c) * p.ldb + k0;
      if constexpr (VEC) {
        // Host guarantees K % 32 == 0, ldb % 16 == 0 and a 16-byte aligned b.
        f.b[c] = (col0 + c < p.N) ? *reinterpret_cast<const v4i*>(bp) : v4i{0, 0, 0, 0};
      } else {
        v4i w = {0, 0, 0, 0};
#pragma unroll
        for (int i = 0; i < 16; ++i)
          if (i < krem && col0 + c < p.N) w[i >> 2] |= (int)((uint32_t)bp[i] << (8 * (i & 3)));
        f.b[c] = w;
      }
    }
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

__device__ __forceinline__ float activate(float x, int act) {
  if (act == VOID_ACT_RELU) return fmaxf(x, 0.0f);
  if (act == VOID_ACT_GELU) {
    // fusion.py:38-43: inner = 0.7978845608 (x + 0.044715 x^3); tanh = 2 sigmoid(2 inner) - 1
    const float inner = 0.7978845608f * (x + 0.044715f * x * x * x);
    const float sig = 1.0f / (1.0f + expf(-2.0f * inner));
    return x * 0.5f * (1.0f + (2.0f * sig - 1.0f));
  }
  if (act == VOID_ACT_SILU) return x * (1.0f / (1.0f + expf(-x)));
  return x;
}

__device__ __forceinline__ uint32_t f32_to_bf16_bits(float x) {
  const uint32_t u = __float_as_uint(x);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;  // quiet NaN
  return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;                  // round to nearest even
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

template <int ELT, int EPI, int OUT, bool BCOL, bool VEC>
__global__ __launch_bounds__(kThreads) void spmm_bsr_kernel(Params p) {
  using A = Accum<ELT, EPI>;
  using Reg = typename A::Reg;
  constexpr bool kInt = A::kInt;

  __shared__ v4i red[kWaves][kTile][kPanel / 4];  // 64 KB: per-wave 32 x 128 partials
  __shared__ int s_last;

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int j = lane & 31, g = lane >> 5;

  const int L = xcd_remap((int)blockIdx.x, (int)gridDim.x);
  const int item_idx = L / p.n_panels;
  const int panel = L - item_idx * p.n_panels;
  const void_work_item it = p.items[item_idx];
  const int col0 = panel * kPanel + j * kColsPerLane;

  Reg acc[kColsPerLane];
#pragma unroll
  for (int c = 0; c < kColsPerLane; ++c) acc[c] = Reg{};

  // Software pipeline: the next tile's loads are in flight while the current
  // tile's MFMAs run.
  int t = it.begin + wave;
  Frag cur, nxt;
  if (t < it.end) load_frag<BCOL, VEC>(p, t, j, g, col0, cur);
  while (t < it.end) {
    const int tn = t + kWaves;
    if (tn < it.end) load_frag<BCOL, VEC>(p, tn, j, g, col0, nxt);
    const float s = (EPI == VOID_EPI_PER_BLOCK) ? (p.per_tensor_a ? p.a_scale[0] : p.a_scale[t]) : 0.f;
    A::step(acc, cur, s);
    cur = nxt;
    t = tn;
  }

  // Cross-wave reduction.  MFMA 32x32 result layout: lane l, register r holds
  // row 8*(r/4) + 4*(l/32) + r%4 of virtual column l%32.
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int row = 8 * (r >> 2) + 4 * g + (r & 3);
    v4i w;
#pragma unroll
    for (int c = 0; c < kColsPerLane; ++c) w[c] = kInt ? (int)acc[c][r] : __float_as_int((float)acc[c][r]);
    red[wave][row][j] = w;
  }
  __syncthreads();

  // Epilogue ownership: wave w finishes rows [8w, 8w+8); lane owns columns
  // col0 .. col0+3 (same j as above) of rows 8w + g + 2i.
  constexpr int kRowsPerWave = kTile / kWaves;
  v4i sumi[kRowsPerWave / 2];
  v4f sumf[kRowsPerWave / 2];
#pragma unroll
  for (int i = 0; i < kRowsPerWave / 2; ++i) {
    const int row = wave * kRowsPerWave + 2 * i + g;
    v4i si = {0, 0, 0, 0};
    v4f sf = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const v4i x = red[w][row][j];
      if constexpr (kInt) si += x;
      else sf += v4f{__int_as_float(x[0]), __int_as_float(x[1]), __int_as_float(x[2]), __int_as_float(x[3])};
    }
    sumi[i] = si;
    sumf[i] = sf;
  }

  if (it.tile >= 0) {
    // Split row: publish this chunk's partial tile, count arrivals, and let
    // the last chunk reduce all partials in chunk order.
    const size_t tile_elems = (size_t)kTile * kPanel;
    v4i* part = static_cast<v4i*>(p.partials);
#pragma unroll
    for (int i = 0; i < kRowsPerWave / 2; ++i) {
      const int row = wave * kRowsPerWave + 2 * i + g;
      const size_t off = ((size_t)(it.slot + it.chunk) * p.n_panels + panel) * tile_elems + (size_t)row * kPanel;
      v4i w;
      if constexpr (kInt) w = sumi[i];
      else w = v4i{__float_as_int(sumf[i][0]), __float_as_int(sumf[i][1]), __float_as_int(sumf[i][2]), __float_as_int(sumf[i][3])};
      part[(off >> 2) + j] = w;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    __syncthreads();
    unsigned* ctr = p.counters + (size_t)it.tile * p.n_panels + panel;
    if (tid == 0) {
      const unsigned old = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
      s_last = (old == (unsigned)(it.nchunks - 1));
    }
    __syncthreads();
    if (!s_last) return;
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    if (tid == 0) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
    for (int i = 0; i < kRowsPerWave / 2; ++i) {
      const int row = wave * kRowsPerWave + 2 * i + g;
      v4i si = {0, 0, 0, 0};
      v4f sf = {0.f, 0.f, 0.f, 0.f};
      for (int ch = 0; ch < it.nchunks; ++ch) {
        const size_t off = ((size_t)(it.slot + ch) * p.n_panels + panel) * tile_elems + (size_t)row * kPanel;
        const v4i x = __builtin_nontemporal_load(&part[(off >> 2) + j]);
        if constexpr (kInt) si += x;
        else sf += v4f{__int_as_float(x[0]), __int_as_float(x[1]), __int_as_float(x[2]), __int_as_float(x[3])};
      }
      sumi[i] = si;
      sumf[i] = sf;
    }
  }

  // Per-column B scale of this lane's four columns.
  float sb[4];
#pragma unroll
  for (int c = 0; c < 4; ++c)
    sb[c] = p.b_scale_vec ? (col0 + c < p.N ? p.b_scale_vec[col0 + c] : 0.f) : p.b_scale;

  float mul[4] = {1.f, 1.f, 1.f, 1.f};
  if constexpr (EPI == VOID_EPI_ROW_MEAN) {
    // int_quant.py:519-526: S = sum fl(s_a * s_b) in tile order, then S / n.
    const int rb = p.row_ptr[it.row], re = p.row_ptr[it.row + 1];
    float S[4] = {0.f, 0.f, 0.f, 0.f};
    for (int tt = rb; tt < re; ++tt) {
      const float sa = p.per_tensor_a ? p.a_scale[0] : p.a_scale[tt];
#pragma unroll
      for (int c = 0; c < 4; ++c) S[c] = __fadd_rn(S[c], __fmul_rn(sa, sb[c]));
    }
    const float n = (float)(re - rb);
#pragma unroll
    for (int c = 0; c < 4; ++c) mul[c] = (re > rb) ? __fdiv_rn(S[c], n) : 0.f;
  } else if constexpr (EPI == VOID_EPI_PER_BLOCK) {
#pragma unroll
    for (int c = 0; c < 4; ++c) mul[c] = sb[c];
  }
  float bias[4] = {0.f, 0.f, 0.f, 0.f};
  if (p.bias) {
#pragma unroll
    for (int c = 0; c < 4; ++c) bias[c] = (col0 + c < p.N) ? p.bias[col0 + c] : 0.f;
  }

#pragma unroll
  for (int i = 0; i < kRowsPerWave / 2; ++i) {
    const int row = wave * kRowsPerWave + 2 * i + g;
    const int grow = it.row * kTile + row;
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

template <int ELT, int EPI, int OUT, bool BCOL, bool VEC>
int launch(const Params& p, int grid, hipStream_t stream) {
  hipLaunchKernelGGL((spmm_bsr_kernel<ELT, EPI, OUT, BCOL, VEC>), dim3(grid), dim3(kThreads), 0, stream, p);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(VOID_ERR_HIP, "kernel launch failed: %s", hipGetErrorString(e));
  return VOID_OK;
}

template <int ELT, int EPI, int OUT>
int launch_layout(const Params& p, int grid, hipStream_t s, bool bcol, bool vec) {
  if (bcol) return vec ? launch<ELT, EPI, OUT, true, true>(p, grid, s) : launch<ELT, EPI, OUT, true, false>(p, grid, s);
  return vec ? launch<ELT, EPI, OUT, false, true>(p, grid, s) : launch<ELT, EPI, OUT, false, false>(p, grid, s);
}

template <int ELT, int EPI>
int launch_out(const Params& p, int grid, hipStream_t s, bool bcol, bool vec, int out) {
  switch (out) {
    case VOID_DT_F32: return launch_layout<ELT, EPI, VOID_DT_F32>(p, grid, s, bcol, vec);
    case VOID_DT_BF16: return launch_layout<ELT, EPI, VOID_DT_BF16>(p, grid, s, bcol, vec);
    case VOID_DT_F16: return launch_layout<ELT, EPI, VOID_DT_F16>(p, grid, s, bcol, vec);
    default: return fail(VOID_ERR_UNSUPPORTED, "out_dtype %d not supported with this epilogue", out);
  }
}

size_t counters_bytes(int32_t n_split_tiles, int32_t n_panels) {
  return ((size_t)n_split_tiles * n_panels * sizeof(unsigned) + 255) & ~(size_t)255;
}

int n_panels_for(int32_t N) { return (N + kPanel - 1) / kPanel; }

int run(int elt, const void_bsr_desc* a, const void_dense_args* d, int32_t epilogue,
        const void_plan* plan, void* workspace, size_t workspace_bytes, hipStream_t stream) {
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
  if (a->n_blocks > 0 && (!a->tiles || !a->col_idx || !a->scales || !d->b))
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
  p.items = items;
  if (n_split_tiles > 0) {
    if (!workspace) return fail(VOID_ERR_WORKSPACE, "plan splits rows but workspace is null");
    const size_t need = void_workspace_bytes(n_split_tiles, plan->n_slots, d->N);
    if (workspace_bytes < need)
      return fail(VOID_ERR_WORKSPACE, "workspace of %zu bytes, plan needs %zu", workspace_bytes, need);
    p.counters = static_cast<unsigned*>(workspace);
    p.partials = static_cast<char*>(workspace) + counters_bytes(n_split_tiles, n_panels);
  }

  const uintptr_t bu = (uintptr_t)d->b, cu = (uintptr_t)d->c;
  const bool c_ok = (cu % 16 == 0) && (d->ldc % 4 == 0) && (d->N % 4 == 0);
  bool vec;
  if (d->b_col_major)
    vec = c_ok && (bu % 16 == 0) && (d->ldb % 16 == 0) && (a->K % kTile == 0);
  else
    vec = c_ok && (bu % 4 == 0) && (d->ldb % 4 == 0);
  const bool bcol = d->b_col_major != 0;
  const int grid = (int)grid64;

  if (elt == kEltI8) {
    switch (epilogue) {
      case VOID_EPI_RAW_I32:
        return bcol ? (vec ? launch<kEltI8, VOID_EPI_RAW_I32, VOID_DT_I32, true, true>(p, grid, stream)
                           : launch<kEltI8, VOID_EPI_RAW_I32, VOID_DT_I32, true, false>(p, grid, stream))
                    : (vec ? launch<kEltI8, VOID_EPI_RAW_I32, VOID_DT_I32, false, true>(p, grid, stream)
                           : launch<kEltI8, VOID_EPI_RAW_I32, VOID_DT_I32, false, false>(p, grid, stream));
      case VOID_EPI_ROW_MEAN:
        return launch_out<kEltI8, VOID_EPI_ROW_MEAN>(p, grid, stream, bcol, vec, d->out_dtype);
      default:
        return launch_out<kEltI8, VOID_EPI_PER_BLOCK>(p, grid, stream, bcol, vec, d->out_dtype);
    }
  }
  return launch_out<kEltFp8, VOID_EPI_PER_BLOCK>(p, grid, stream, bcol, vec, d->out_dtype);
}

}  // namespace

extern "C" {

int void_abi_version(void) { return VOID_AMD_ABI_VERSION; }

const char* void_last_error(void) { return g_err; }

int void_panel_width(void) { return kPanel; }

int void_streamk_plan(const int32_t* row_ptr, int32_t n_block_rows, int32_t chunk_tiles,
                      void_work_item* items, int32_t capacity, int32_t* n_items,
                      int32_t* n_split_tiles, int32_t* n_slots) {
  g_err[0] = 0;
  if (!row_ptr || !n_items || !n_split_tiles || !n_slots || n_block_rows < 0 || chunk_tiles < 1)
    return fail(VOID_ERR_ARG, "bad planner arguments");
  std::vector<void_work_item> out;
  out.reserve(n_block_rows);
  int32_t tiles = 0, slots = 0;
  for (int32_t r = 0; r < n_block_rows; ++r) {
    const int32_t b = row_ptr[r], e = row_ptr[r + 1];
    if (e < b) return fail(VOID_ERR_ARG, "row_ptr decreases at row %d", r);
    const int32_t n = e - b;
    if (n <= chunk_tiles) {
      out.push_back(void_work_item{r, b, e, -1, 1, 0, 0, 0});
      continue;
    }
    const int32_t nch = (n + chunk_tiles - 1) / chunk_tiles;
    for (int32_t c = 0; c < nch; ++c) {
      const int32_t cb = b + (int32_t)((int64_t)c * n / nch);
      const int32_t ce = b + (int32_t)((int64_t)(c + 1) * n / nch);
      out.push_back(void_work_item{r, cb, ce, tiles, nch, c, slots, 0});
    }
    tiles += 1;
    slots += nch;
  }
  // Longest items first so that the tail of the dispatch is short ones.
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

int void_spmm_fp8(const void_bsr_desc* a, const void_dense_args* d, const void_plan* plan,
                  void* workspace, size_t workspace_bytes, hipStream_t stream) {
  return run(kEltFp8, a, d, VOID_EPI_PER_BLOCK, plan, workspace, workspace_bytes, stream);
}

}  // extern "C"
