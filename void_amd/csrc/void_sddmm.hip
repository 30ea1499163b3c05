// void_sddmm.hip — gradient of the SpMM with respect to the nonzero tiles of
// A (void_spmm_backward_a_kernel, void/autograd.py:14-97), declared in
// include/void_amd.h:
//
//   grad[t] = dC[32 br_t .. +32, :] @ B[32 bc_t .. +32, :]^T     (32 x 32)
//
// for every active tile t — a sampled dense-dense product on the tiles'
// support.  One workgroup of 4 wave64s per tile: wave w reduces the chunks
// w, w+4, ... of 32 columns of N on v_mfma_f32_32x32x2_f32 (exact fp32
// products, fp32 accumulation), and the four partial 32x32 blocks are summed
// through LDS in wave order.  Within a chunk lane (i, g) loads 16 consecutive
// values of row i of each operand (n = n0 + 16g .. +15) and MFMA s (s < 16)
// takes n = n0 + 16g + s from both, so the reduction order agrees for the two
// operands.  The loads of a wave's next chunk are in flight during the 16
// MFMAs of the current one.
// Rows past M (of dC) or K (of B) and columns past N read as zero, as the
// reference's boundary-checked loads do.

#include <hip/hip_runtime.h>

#include <climits>
#include <cstdint>
#include <cstdlib>
#include <cstring>

#include "void_amd.h"
#include "lds_dma.h"

extern "C" __attribute__((visibility("hidden"))) int void_internal_fail(int code, const char* msg);

namespace {

constexpr int kT = 32;
constexpr int kWaves = 4;  // waves per tile, each a quarter of the chunks of N

typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef _Float16 v8hf __attribute__((ext_vector_type(8)));

struct Chunk {
  v4f x[4];  // dC[row_x][n0 + 16g + 4q .. +3]
  v4f y[4];  // B[row_y][n0 + 16g + 4q .. +3]
};

__device__ __forceinline__ uint32_t bf16_bits(float x) {
  const uint32_t u = __float_as_uint(x);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
  return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}

// VEC: ldg, ldb and N multiples of 4 and 16-byte aligned operands, so a
// 4-column group is either wholly inside N or wholly past it.
template <int OUT, bool VEC>
__global__ __launch_bounds__(64 * kWaves) void sddmm_kernel(
    const float* __restrict__ dC, int64_t ldg, const float* __restrict__ B, int64_t ldb,
    const int32_t* __restrict__ block_rows, const int32_t* __restrict__ block_cols, int32_t n_blocks, int32_t M,
    int32_t N, int32_t K, void* __restrict__ grad) {
  __shared__ float part[kWaves][16][64];  // [wave][register][lane]: conflict-free writes and reads
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t t = blockIdx.x;
  const int i = lane & 31, g = lane >> 5;
  const int br = block_rows[t], bc = block_cols[t];
  const int rx = br * kT + i, ry = bc * kT + i;
  const bool okx = rx < M, oky = ry < K;
  const float* xrow = dC + (int64_t)(okx ? rx : 0) * ldg;
  const float* yrow = B + (int64_t)(oky ? ry : 0) * ldb;
  const int n_chunks = (N + kT - 1) / kT;

  auto load = [&](Chunk& c, int chunk) {
    const int nb = chunk * kT + 16 * g;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int n = nb + 4 * q;
      if constexpr (VEC) {
        const bool in = n < N;
        const int nn = in ? n : 0;
        v4f vx = *reinterpret_cast<const v4f*>(xrow + nn);
        v4f vy = *reinterpret_cast<const v4f*>(yrow + nn);
        c.x[q] = (in && okx) ? vx : v4f{0.f, 0.f, 0.f, 0.f};
        c.y[q] = (in && oky) ? vy : v4f{0.f, 0.f, 0.f, 0.f};
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const bool in = n + e < N;
          const int nn = in ? n + e : 0;
          const float vx = xrow[nn], vy = yrow[nn];
          c.x[q][e] = (in && okx) ? vx : 0.f;
          c.y[q][e] = (in && oky) ? vy : 0.f;
        }
      }
    }
  };
  v16f acc = {};
  auto consume = [&](const Chunk& c) {
#pragma unroll
    for (int s = 0; s < 16; ++s) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(c.x[s >> 2][s & 3], c.y[s >> 2][s & 3], acc, 0, 0, 0);
  };
  if (wave < n_chunks) {
    // This wave's chunks: wave, wave + 4, ...; the next one is loaded
    // unconditionally (past the end it re-reads the current one), which keeps
    // the vmcnt waits exact.
    Chunk X, Y;
    load(X, wave);
    for (int ch = wave;;) {
      load(Y, ch + kWaves < n_chunks ? ch + kWaves : ch);
      consume(X);
      ch += kWaves;
      if (ch >= n_chunks) break;
      load(X, ch + kWaves < n_chunks ? ch + kWaves : ch);
      consume(Y);
      ch += kWaves;
      if (ch >= n_chunks) break;
    }
  }
#pragma unroll
  for (int r = 0; r < 16; ++r) part[wave][r][lane] = acc[r];
  __syncthreads();
  // Wave w sums registers 4w .. 4w+3 over the four waves, in wave order, and
  // stores them: lane (j, g), register r is tile row 8 (r / 4) + 4 g + r % 4,
  // column j.
  const int j = lane & 31;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int r = 4 * wave + q;
    float v = part[0][r][lane];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) v += part[w][r][lane];
    const int row = 8 * (r >> 2) + 4 * g + (r & 3);
    const int64_t off = t * (kT * kT) + row * kT + j;
    if constexpr (OUT == VOID_DT_F32) static_cast<float*>(grad)[off] = v;
    else if constexpr (OUT == VOID_DT_BF16) static_cast<uint16_t*>(grad)[off] = (uint16_t)bf16_bits(v);
    else {
      _Float16 h = (_Float16)v;
      uint16_t u;
      __builtin_memcpy(&u, &h, 2);
      static_cast<uint16_t*>(grad)[off] = u;
    }
  }
}

template <int OUT, bool VEC>
int go(const float* dC, int64_t ldg, const float* B, int64_t ldb, const int32_t* rows, const int32_t* cols,
       int32_t n, int32_t M, int32_t N, int32_t K, void* grad, hipStream_t stream) {
  hipLaunchKernelGGL((sddmm_kernel<OUT, VEC>), dim3(n), dim3(64 * kWaves), 0, stream, dC, ldg, B, ldb, rows,
                     cols, n, M, N, K, grad);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return void_internal_fail(VOID_ERR_HIP, hipGetErrorString(e));
  return VOID_OK;
}

// Row-grouped variant (void_sddmm_rows_f32): the tiles of one block-row
// share their dC rows, so one workgroup of kGW waves takes up to kGW tiles
// of a block-row (a group).  Per chunk of 32 columns of N the workgroup
// stages the group's dC block [32 x 32] once in LDS (double-buffered), and
// each wave streams its own tile's B rows one chunk ahead in registers and
// runs the chunk's 16 MFMAs with the A operand read from LDS.  dC is then
// read once per group instead of once per tile.
constexpr int kGW = 8;
constexpr int kXPad = 36;  // floats per staged dC row: lanes i and i + 2 land on other banks

template <int OUT, bool VEC>
__global__ __launch_bounds__(64 * kGW) void sddmm_rows_kernel(
    const float* __restrict__ dC, int64_t ldg, const float* __restrict__ B, int64_t ldb,
    const int32_t* __restrict__ groups, const int32_t* __restrict__ col_idx, const int64_t* __restrict__ tile_index,
    int32_t M, int32_t N, int32_t K, void* __restrict__ grad) {
  __shared__ __attribute__((aligned(16))) float xs[2][kT][kXPad];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int i = lane & 31, g = lane >> 5;
  const int br = groups[3 * blockIdx.x], pos0 = groups[3 * blockIdx.x + 1], cnt = groups[3 * blockIdx.x + 2];
  const bool has = wave < cnt;
  const int bc = has ? col_idx[pos0 + wave] : 0;
  const int64_t out_t = has ? (tile_index ? tile_index[pos0 + wave] : (int64_t)(pos0 + wave)) : 0;
  const int n_chunks = (N + kT - 1) / kT;

  // dC staging: thread tid moves row tid / 16, columns 2 (tid % 16) .. +1.
  const int xr = tid >> 4, xc = 2 * (tid & 15);
  const int grow = br * kT + xr;
  const bool okx = grow < M;
  const float* xsrc = dC + (int64_t)(okx ? grow : 0) * ldg;
  // B rows of this wave's tile: lane (i, g) takes row i, columns 16 g .. +15.
  const int ry = bc * kT + i;
  const bool oky = has && ry < K;
  const float* yrow = B + (int64_t)(oky ? ry : 0) * ldb;

  auto load_x = [&](int ch, float& a, float& b2) {
    const int n = ch * kT + xc;
    if constexpr (VEC) {
      const bool in = n < N;  // N even here, so a pair is wholly in or out
      const float2 v = *reinterpret_cast<const float2*>(xsrc + (in ? n : 0));
      a = (in && okx) ? v.x : 0.f;
      b2 = (in && okx) ? v.y : 0.f;
    } else {
      const float v0 = xsrc[n < N ? n : 0], v1 = xsrc[n + 1 < N ? n + 1 : 0];
      a = (n < N && okx) ? v0 : 0.f;
      b2 = (n + 1 < N && okx) ? v1 : 0.f;
    }
  };
  auto load_y = [&](int ch, v4f (&y)[4]) {
    const int nb = ch * kT + 16 * g;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int n = nb + 4 * q;
      if constexpr (VEC) {
        const bool in = n < N;
        const v4f v = *reinterpret_cast<const v4f*>(yrow + (in ? n : 0));
        y[q] = (in && oky) ? v : v4f{0.f, 0.f, 0.f, 0.f};
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const bool in = n + e < N;
          const float v = yrow[in ? n + e : 0];
          y[q][e] = (in && oky) ? v : 0.f;
        }
      }
    }
  };

  v16f acc = {};
  v4f y0[4], y1[4];
  float xa, xb;
  load_x(0, xa, xb);
  load_y(0, y0);
  xs[0][xr][xc] = xa;
  xs[0][xr][xc + 1] = xb;
  __syncthreads();
  for (int ch = 0; ch < n_chunks; ++ch) {
    const bool more = ch + 1 < n_chunks;
    if (more) {
      load_x(ch + 1, xa, xb);
      load_y(ch + 1, y1);
    }
    if (has) {
      const float* xrow = &xs[ch & 1][i][16 * g];
      v4f x[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) x[q] = *reinterpret_cast<const v4f*>(xrow + 4 * q);
#pragma unroll
      for (int s2 = 0; s2 < 16; ++s2)
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(x[s2 >> 2][s2 & 3], y0[s2 >> 2][s2 & 3], acc, 0, 0, 0);
    }
    if (more) {
      xs[(ch + 1) & 1][xr][xc] = xa;
      xs[(ch + 1) & 1][xr][xc + 1] = xb;
    }
    __syncthreads();  // chunk ch + 1 staged; every wave is done with chunk ch's buffer
#pragma unroll
    for (int q = 0; q < 4; ++q) y0[q] = y1[q];
  }
  if (!has) return;
  // Lane (j, g), register r: tile row 8 (r / 4) + 4 g + r % 4, column j.
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int row = 8 * (r >> 2) + 4 * g + (r & 3);
    const int64_t off = out_t * (kT * kT) + row * kT + i;
    const float v = acc[r];
    if constexpr (OUT == VOID_DT_F32) static_cast<float*>(grad)[off] = v;
    else if constexpr (OUT == VOID_DT_BF16) static_cast<uint16_t*>(grad)[off] = (uint16_t)bf16_bits(v);
    else {
      _Float16 h = (_Float16)v;
      uint16_t u;
      __builtin_memcpy(&u, &h, 2);
      static_cast<uint16_t*>(grad)[off] = u;
    }
  }
}

// Row-grouped SDDMM on an LDS-DMA ring (void_sddmm_rows_f32 with 16-byte
// aligned operands).  One workgroup of 8 waves per group of up to 8 tiles of
// one block-row, wave w on tile w, as above; the reduction over N runs in
// chunks of 32 columns, double-buffered in LDS.  A stage holds the group's
// dC block (32 rows x 32 columns, 4 KB) and each tile's B block (4 KB),
// loaded by buffer_load ... lds: every wave issues exactly 5 loads per stage
// (the four 8-row parts of its tile's B block and one part of dC, or a
// dummy load at kOutOfRange for waves 4-7), so the waits are fixed vmcnt
// counts.  Rows are 128 bytes; the 16-byte segment s of row r sits at
// position s ^ (r & 7), so that the 8 rows an 8-lane read phase touches fall
// on distinct banks.  Lane (i, g) reads row i, columns 16 g .. 16 g + 15 of
// both blocks (four 16-byte LDS reads each) and MFMA s takes column
// 16 g + s from both operands.  Two 72 KB workgroups per CU move 72 KB per
// chunk for 4096 cycles of MFMA per SIMD, below the L2 -> LDS rate, so the
// matrix cores bound the loop.  Against 16-column chunks in rings of 3 or 4
// stages, and 32-column chunks in 3 stages (one workgroup per CU), this
// shape measured fastest on c2, c3 and c5.
constexpr int kRW = 8;    // waves per workgroup, one tile each
constexpr int kRing = 2;  // stages (double buffer)

// Block geometry of a ring with CW columns of N per chunk: 16-byte segments
// per block row, rows per 1 KB load, loads per 32-row block, block bytes.
template <int CW>
struct RingGeo {
  static constexpr int kSegs = CW / 4;
  static constexpr int kRowsPerLoad = 64 / kSegs;
  static constexpr int kLoadsPerBlk = kT / kRowsPerLoad;
  static constexpr int kBlk = kT * CW * 4;
  // Segment s of block row r sits at position s ^ swz(r), so that the 8 rows
  // of an 8-lane read phase fall on distinct banks.
  __device__ static __forceinline__ int swz(int r) { return kSegs == 8 ? (r & 7) : ((r >> 1) & 3); }
};

// PER_TILE (void_sddmm_f32, tiles in any order): wave w takes tile 8 b + w
// of workgroup b with a dC block of its own; a stage holds each wave's dC
// and B blocks of a 16-column chunk (32 KB, 64 KB double-buffered, two
// workgroups per CU), 4 loads per wave.
//
// IN = VOID_DT_BF16 / VOID_DT_F16 (void_sddmm_rows_bf16 / _f16): 16-bit dC and
// B with the same byte geometry, so a chunk holds twice the columns; lane
// (i, g) feeds v_mfma_f32_32x32x16_{bf16,f16} q with its q-th 16-byte segment
// (8 consecutive n) of row i of both operands, whose products are exact in
// fp32 as on the fp32 MFMA.
template <int OUT, bool PER_TILE, int IN = VOID_DT_F32>
__global__ __launch_bounds__(64 * kRW) void sddmm_ring_kernel(
    const void* __restrict__ dC, int64_t ldg, const void* __restrict__ B, int64_t ldb,
    const int32_t* __restrict__ groups, const int32_t* __restrict__ col_idx, const int64_t* __restrict__ tile_index,
    const int32_t* __restrict__ block_rows, const int32_t* __restrict__ block_cols, int32_t n_blocks,
    int32_t M, int32_t N, int32_t K, void* __restrict__ grad) {
  constexpr int kEsz = IN == VOID_DT_F32 ? 4 : 2;
  constexpr int kCW4 = PER_TILE ? 16 : 32;  // chunk width in 4-byte words
  constexpr int kCW = kCW4 * 4 / kEsz;      // columns of N per chunk
  constexpr int kEps = 16 / kEsz;           // columns per 16-byte segment
  using Geo = RingGeo<kCW4>;
  constexpr int kSegs = Geo::kSegs, kRowsPerLoad = Geo::kRowsPerLoad, kLoadsPerBlk = Geo::kLoadsPerBlk;
  constexpr int kBlk = Geo::kBlk;
  constexpr int kStage = PER_TILE ? 2 * kRW * kBlk : (1 + kRW) * kBlk;
  constexpr int kRingJunk = kRing * kStage;  // 1 KB that the dummy dC loads fill
  constexpr int kLoadsPerStage = PER_TILE ? 2 * kLoadsPerBlk : kLoadsPerBlk + 1;
  static_assert(kLoadsPerBlk <= kRW, "the shared dC block's loads go one per wave");
  static_assert(kRing >= 2 && kRing <= 4, "stage waits cover up to two stages ahead");
  __shared__ __attribute__((aligned(16))) uint8_t smem[kRingJunk + 1024];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int i = lane & 31, g = lane >> 5;
  bool has;
  int br, bc;
  int64_t out_t;
  if constexpr (PER_TILE) {
    const int64_t t = (int64_t)blockIdx.x * kRW + wave;
    has = t < n_blocks;
    br = has ? block_rows[t] : 0;
    bc = has ? block_cols[t] : 0;
    out_t = t;
  } else {
    br = groups[3 * blockIdx.x];
    const int pos0 = groups[3 * blockIdx.x + 1], cnt = groups[3 * blockIdx.x + 2];
    has = wave < cnt;
    bc = has ? col_idx[pos0 + wave] : 0;
    out_t = has ? (tile_index ? tile_index[pos0 + wave] : (int64_t)(pos0 + wave)) : 0;
  }
  const int n_chunks = (N + kCW - 1) / kCW;
  // This wave's blocks within a stage.
  const int xoff = PER_TILE ? 2 * wave * kBlk : 0;
  const int yoff = PER_TILE ? (2 * wave + 1) * kBlk : (1 + wave) * kBlk;

  // Load lane l of part h: row kRowsPerLoad h + l / kSegs, LDS position
  // l % kSegs holding source segment (l % kSegs) ^ swz(row).  Rows past M
  // (dC) or K (B), and segments past N (N is a multiple of 4 here), read
  // zeros.
  const v4s rx = sgpr_rsrc(static_cast<const char*>(dC) + (int64_t)br * kT * ldg * kEsz),
            ry = sgpr_rsrc(static_cast<const char*>(B) + (int64_t)bc * kT * ldb * kEsz);
  int vy[kLoadsPerBlk], vx[kLoadsPerBlk], sg[kLoadsPerBlk];
#pragma unroll
  for (int h = 0; h < kLoadsPerBlk; ++h) {
    // Grouped: wave w loads only part w of the shared dC block.
    const int hx = PER_TILE ? h : wave % kLoadsPerBlk;
    const int row = kRowsPerLoad * h + lane / kSegs;
    const int xrow = kRowsPerLoad * hx + lane / kSegs;
    sg[h] = (lane % kSegs) ^ Geo::swz(row);
    vy[h] = has && bc * kT + row < K ? row * (int)ldb * kEsz + sg[h] * 16 : kOutOfRange;
    const bool x_live = PER_TILE ? has : wave < kLoadsPerBlk;
    vx[h] = x_live && br * kT + xrow < M ? xrow * (int)ldg * kEsz + ((lane % kSegs) ^ Geo::swz(xrow)) * 16 : kOutOfRange;
  }
  auto issue = [&](int ch) {
    uint8_t* st = smem + (ch % kRing) * kStage;
    const int n0 = ch * kCW;
#pragma unroll
    for (int h = 0; h < kLoadsPerBlk; ++h)
      dma_b128(ry, st + yoff + h * 1024, n0 + kEps * sg[h] < N ? vy[h] : kOutOfRange, n0 * kEsz);
    if constexpr (PER_TILE) {
#pragma unroll
      for (int h = 0; h < kLoadsPerBlk; ++h)
        dma_b128(rx, st + xoff + h * 1024, n0 + kEps * sg[h] < N ? vx[h] : kOutOfRange, n0 * kEsz);
    } else {
      // The dC part's rows lie whole 8-row groups from part 0's, and with 8
      // segments per row the swizzle depends only on the row mod 8, so
      // sg[0] is this lane's dC segment too.
      const bool x_wave = wave < kLoadsPerBlk;
      dma_b128(rx, x_wave ? st + wave * 1024 : smem + kRingJunk, n0 + kEps * sg[0] < N ? vx[0] : kOutOfRange,
               n0 * kEsz);
    }
  };

  // Lane (i, g): row i, source segments kSegs / 2 g .. + kSegs / 2 - 1.
  constexpr int kHalf = kSegs / 2;
  int rd[kHalf];
#pragma unroll
  for (int q = 0; q < kHalf; ++q) rd[q] = i * (kCW4 * 4) + (((kHalf * g + q) ^ Geo::swz(i)) << 4);
  v16f acc = {};
#pragma unroll
  for (int k = 0; k < kRing - 1; ++k)
    if (k < n_chunks) issue(k);
  for (int ch = 0; ch < n_chunks; ++ch) {
    wait_stages<kLoadsPerStage>(min(n_chunks - 1, ch + kRing - 2) - ch);
    // Every wave's part of chunk ch has landed, and every wave has finished
    // reading chunk ch - 1, whose slot the next issue overwrites.
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    if (ch + kRing - 1 < n_chunks) issue(ch + kRing - 1);
    if (has) {
      const uint8_t* st = smem + (ch % kRing) * kStage;
      v4f x[kHalf], y[kHalf];
#pragma unroll
      for (int q = 0; q < kHalf; ++q) {
        x[q] = *reinterpret_cast<const v4f*>(st + xoff + rd[q]);
        y[q] = *reinterpret_cast<const v4f*>(st + yoff + rd[q]);
      }
      if constexpr (IN == VOID_DT_F32) {
#pragma unroll
        for (int q = 0; q < kHalf; ++q)
#pragma unroll
          for (int s2 = 0; s2 < 4; ++s2) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(x[q][s2], y[q][s2], acc, 0, 0, 0);
      } else if constexpr (IN == VOID_DT_BF16) {
#pragma unroll
        for (int q = 0; q < kHalf; ++q)
          acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf, x[q]), __builtin_bit_cast(v8bf, y[q]),
                                                        acc, 0, 0, 0);
      } else {
#pragma unroll
        for (int q = 0; q < kHalf; ++q)
          acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8hf, x[q]), __builtin_bit_cast(v8hf, y[q]),
                                                       acc, 0, 0, 0);
      }
    }
  }
  if (!has) return;
  // Lane (j, g), register r: tile row 8 (r / 4) + 4 g + r % 4, column j.
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int row = 8 * (r >> 2) + 4 * g + (r & 3);
    const int64_t off = out_t * (kT * kT) + row * kT + i;
    const float v = acc[r];
    if constexpr (OUT == VOID_DT_F32) static_cast<float*>(grad)[off] = v;
    else if constexpr (OUT == VOID_DT_BF16) static_cast<uint16_t*>(grad)[off] = (uint16_t)bf16_bits(v);
    else {
      _Float16 h = (_Float16)v;
      uint16_t u;
      __builtin_memcpy(&u, &h, 2);
      static_cast<uint16_t*>(grad)[off] = u;
    }
  }
}

// The ring kernels need 16-byte rows (VEC) and 31-bit offsets within 32
// rows of either operand; VOID_AMD_SDDMM=rows keeps the register-staged
// kernels.
bool use_ring(bool vec, int64_t ldg, int64_t ldb) {
  const char* force = getenv("VOID_AMD_SDDMM");
  return vec && !(force && strcmp(force, "rows") == 0) && (int64_t)kT * ldg * 4 < INT32_MAX &&
         (int64_t)kT * ldb * 4 < INT32_MAX;
}

// void_sddmm_f32: the per-tile ring where the operands allow, else one
// workgroup per tile on the register-staged kernel.
template <int OUT, bool VEC>
int go_tiles(const float* dC, int64_t ldg, const float* B, int64_t ldb, const int32_t* rows, const int32_t* cols,
             int32_t n, int32_t M, int32_t N, int32_t K, void* grad, hipStream_t stream) {
  if (!use_ring(VEC, ldg, ldb)) return go<OUT, VEC>(dC, ldg, B, ldb, rows, cols, n, M, N, K, grad, stream);
  hipLaunchKernelGGL((sddmm_ring_kernel<OUT, true>), dim3((n + kRW - 1) / kRW), dim3(64 * kRW), 0, stream, dC, ldg, B,
                     ldb, nullptr, nullptr, nullptr, rows, cols, n, M, N, K, grad);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return void_internal_fail(VOID_ERR_HIP, hipGetErrorString(e));
  return VOID_OK;
}

template <int OUT, bool VEC>
int go_rows(const float* dC, int64_t ldg, const float* B, int64_t ldb, const int32_t* groups, int32_t n_groups,
            const int32_t* col_idx, const int64_t* tile_index, int32_t M, int32_t N, int32_t K, void* grad,
            hipStream_t stream) {
  if (use_ring(VEC, ldg, ldb))
    hipLaunchKernelGGL((sddmm_ring_kernel<OUT, false>), dim3(n_groups), dim3(64 * kRW), 0, stream, dC, ldg, B, ldb,
                       groups, col_idx, tile_index, nullptr, nullptr, 0, M, N, K, grad);
  else
    hipLaunchKernelGGL((sddmm_rows_kernel<OUT, VEC>), dim3(n_groups), dim3(64 * kGW), 0, stream, dC, ldg, B, ldb,
                       groups, col_idx, tile_index, M, N, K, grad);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return void_internal_fail(VOID_ERR_HIP, hipGetErrorString(e));
  return VOID_OK;
}

// 16-bit operands: the row-grouped ring only (16-byte aligned rows, N % 8
// == 0, 31-bit offsets within 32 rows of either operand).
template <int IN>
int go_rows16(const void* dC, int64_t ldg, const void* B, int64_t ldb, const int32_t* groups, int32_t n_groups,
              const int32_t* col_idx, const int64_t* tile_index, int32_t M, int32_t N, int32_t K, void* grad,
              int32_t out_dtype, hipStream_t stream) {
  const bool ok = ((uintptr_t)dC % 16 == 0) && ((uintptr_t)B % 16 == 0) && ldg % 8 == 0 && ldb % 8 == 0 &&
                  N % 8 == 0 && (int64_t)kT * ldg * 2 < INT32_MAX && (int64_t)kT * ldb * 2 < INT32_MAX;
  if (!ok)
    return void_internal_fail(VOID_ERR_UNSUPPORTED,
                              "16-bit SDDMM needs 16-byte aligned rows (ldg, ldb, N multiples of 8)");
  auto launch = [&](auto k) {
    hipLaunchKernelGGL(k, dim3(n_groups), dim3(64 * kRW), 0, stream, dC, ldg, B, ldb, groups, col_idx, tile_index,
                       nullptr, nullptr, 0, M, N, K, grad);
  };
  switch (out_dtype) {
    case VOID_DT_F32: launch(sddmm_ring_kernel<VOID_DT_F32, false, IN>); break;
    case VOID_DT_BF16: launch(sddmm_ring_kernel<VOID_DT_BF16, false, IN>); break;
    case VOID_DT_F16: launch(sddmm_ring_kernel<VOID_DT_F16, false, IN>); break;
    default: return void_internal_fail(VOID_ERR_UNSUPPORTED, "gradient tiles are f32, bf16 or f16");
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return void_internal_fail(VOID_ERR_HIP, hipGetErrorString(e));
  return VOID_OK;
}

int rows16_args(const void* grad_c, int64_t ldg, const void* b, int64_t ldb, const int32_t* groups, int32_t n_groups,
                const int32_t* col_idx, int32_t M, int32_t N, int32_t K, void* grad_tiles) {
  void_internal_fail(VOID_OK, "");
  if (n_groups < 0 || M < 0 || N < 0 || K < 0) return void_internal_fail(VOID_ERR_ARG, "negative size");
  if (n_groups == 0) return VOID_OK;
  if (!grad_c || !b || !groups || !col_idx || !grad_tiles) return void_internal_fail(VOID_ERR_ARG, "null pointer");
  if (ldg < N || ldb < N) return void_internal_fail(VOID_ERR_ARG, "leading dimension smaller than N");
  if (N == 0) return void_internal_fail(VOID_ERR_ARG, "N = 0: the gradient is zero, fill it instead");
  return VOID_OK;
}

}  // namespace

extern "C" int void_sddmm_rows_bf16(const void* grad_c, int64_t ldg, const void* b, int64_t ldb,
                                    const int32_t* groups, int32_t n_groups, const int32_t* col_idx,
                                    const int64_t* tile_index, int32_t M, int32_t N, int32_t K, void* grad_tiles,
                                    int32_t out_dtype, hipStream_t stream) {
  const int st = rows16_args(grad_c, ldg, b, ldb, groups, n_groups, col_idx, M, N, K, grad_tiles);
  if (st != VOID_OK || n_groups == 0) return st;
  return go_rows16<VOID_DT_BF16>(grad_c, ldg, b, ldb, groups, n_groups, col_idx, tile_index, M, N, K, grad_tiles,
                                 out_dtype, stream);
}

extern "C" int void_sddmm_rows_f16(const void* grad_c, int64_t ldg, const void* b, int64_t ldb,
                                   const int32_t* groups, int32_t n_groups, const int32_t* col_idx,
                                   const int64_t* tile_index, int32_t M, int32_t N, int32_t K, void* grad_tiles,
                                   int32_t out_dtype, hipStream_t stream) {
  const int st = rows16_args(grad_c, ldg, b, ldb, groups, n_groups, col_idx, M, N, K, grad_tiles);
  if (st != VOID_OK || n_groups == 0) return st;
  return go_rows16<VOID_DT_F16>(grad_c, ldg, b, ldb, groups, n_groups, col_idx, tile_index, M, N, K, grad_tiles,
                                out_dtype, stream);
}

extern "C" int void_sddmm_f32(const float* grad_c, int64_t ldg, const float* b, int64_t ldb,
                              const int32_t* block_rows, const int32_t* block_cols, int32_t n_blocks, int32_t M,
                              int32_t N, int32_t K, void* grad_tiles, int32_t out_dtype, hipStream_t stream) {
  void_internal_fail(VOID_OK, "");
  if (n_blocks < 0 || M < 0 || N < 0 || K < 0) return void_internal_fail(VOID_ERR_ARG, "negative size");
  if (n_blocks == 0) return VOID_OK;
  if (!grad_c || !b || !block_rows || !block_cols || !grad_tiles)
    return void_internal_fail(VOID_ERR_ARG, "null pointer");
  if (ldg < N || ldb < N) return void_internal_fail(VOID_ERR_ARG, "leading dimension smaller than N");
  if (N == 0) return void_internal_fail(VOID_ERR_ARG, "N = 0: the gradient is zero, fill it instead");
  const bool vec = ((uintptr_t)grad_c % 16 == 0) && ((uintptr_t)b % 16 == 0) && ldg % 4 == 0 && ldb % 4 == 0 &&
                   N % 4 == 0;
  switch (out_dtype) {
    case VOID_DT_F32:
      return vec ? go_tiles<VOID_DT_F32, true>(grad_c, ldg, b, ldb, block_rows, block_cols, n_blocks, M, N, K, grad_tiles, stream)
                 : go_tiles<VOID_DT_F32, false>(grad_c, ldg, b, ldb, block_rows, block_cols, n_blocks, M, N, K, grad_tiles, stream);
    case VOID_DT_BF16:
      return vec ? go_tiles<VOID_DT_BF16, true>(grad_c, ldg, b, ldb, block_rows, block_cols, n_blocks, M, N, K, grad_tiles, stream)
                 : go_tiles<VOID_DT_BF16, false>(grad_c, ldg, b, ldb, block_rows, block_cols, n_blocks, M, N, K, grad_tiles, stream);
    case VOID_DT_F16:
      return vec ? go_tiles<VOID_DT_F16, true>(grad_c, ldg, b, ldb, block_rows, block_cols, n_blocks, M, N, K, grad_tiles, stream)
                 : go_tiles<VOID_DT_F16, false>(grad_c, ldg, b, ldb, block_rows, block_cols, n_blocks, M, N, K, grad_tiles, stream);
    default:
      return void_internal_fail(VOID_ERR_UNSUPPORTED, "gradient tiles are f32, bf16 or f16");
  }
}

extern "C" int void_sddmm_rows_f32(const float* grad_c, int64_t ldg, const float* b, int64_t ldb,
                                   const int32_t* groups, int32_t n_groups, const int32_t* col_idx,
                                   const int64_t* tile_index, int32_t M, int32_t N, int32_t K, void* grad_tiles,
                                   int32_t out_dtype, hipStream_t stream) {
  void_internal_fail(VOID_OK, "");
  if (n_groups < 0 || M < 0 || N < 0 || K < 0) return void_internal_fail(VOID_ERR_ARG, "negative size");
  if (n_groups == 0) return VOID_OK;
  if (!grad_c || !b || !groups || !col_idx || !grad_tiles) return void_internal_fail(VOID_ERR_ARG, "null pointer");
  if (ldg < N || ldb < N) return void_internal_fail(VOID_ERR_ARG, "leading dimension smaller than N");
  if (N == 0) return void_internal_fail(VOID_ERR_ARG, "N = 0: the gradient is zero, fill it instead");
  const bool vec = ((uintptr_t)grad_c % 16 == 0) && ((uintptr_t)b % 16 == 0) && ldg % 4 == 0 && ldb % 4 == 0 &&
                   N % 4 == 0;
  switch (out_dtype) {
    case VOID_DT_F32:
      return vec ? go_rows<VOID_DT_F32, true>(grad_c, ldg, b, ldb, groups, n_groups, col_idx, tile_index, M, N, K, grad_tiles, stream)
                 : go_rows<VOID_DT_F32, false>(grad_c, ldg, b, ldb, groups, n_groups, col_idx, tile_index, M, N, K, grad_tiles, stream);
    case VOID_DT_BF16:
      return vec ? go_rows<VOID_DT_BF16, true>(grad_c, ldg, b, ldb, groups, n_groups, col_idx, tile_index, M, N, K, grad_tiles, stream)
                 : go_rows<VOID_DT_BF16, false>(grad_c, ldg, b, ldb, groups, n_groups, col_idx, tile_index, M, N, K, grad_tiles, stream);
    case VOID_DT_F16:
      return vec ? go_rows<VOID_DT_F16, true>(grad_c, ldg, b, ldb, groups, n_groups, col_idx, tile_index, M, N, K, grad_tiles, stream)
                 : go_rows<VOID_DT_F16, false>(grad_c, ldg, b, ldb, groups, n_groups, col_idx, tile_index, M, N, K, grad_tiles, stream);
    default:
      return void_internal_fail(VOID_ERR_UNSUPPORTED, "gradient tiles are f32, bf16 or f16");
  }
}
