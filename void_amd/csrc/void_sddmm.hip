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

#include <cstdint>

#include "void_amd.h"

extern "C" __attribute__((visibility("hidden"))) int void_internal_fail(int code, const char* msg);

namespace {

constexpr int kT = 32;
constexpr int kWaves = 4;  // waves per tile, each a quarter of the chunks of N

typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));

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

}  // namespace

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
      return vec ? go<VOID_DT_F32, true>(grad_c, ldg, b, ldb, block_rows, block_cols, n_blocks, M, N, K, grad_tiles, stream)
                 : go<VOID_DT_F32, false>(grad_c, ldg, b, ldb, block_rows, block_cols, n_blocks, M, N, K, grad_tiles, stream);
    case VOID_DT_BF16:
      return vec ? go<VOID_DT_BF16, true>(grad_c, ldg, b, ldb, block_rows, block_cols, n_blocks, M, N, K, grad_tiles, stream)
                 : go<VOID_DT_BF16, false>(grad_c, ldg, b, ldb, block_rows, block_cols, n_blocks, M, N, K, grad_tiles, stream);
    case VOID_DT_F16:
      return vec ? go<VOID_DT_F16, true>(grad_c, ldg, b, ldb, block_rows, block_cols, n_blocks, M, N, K, grad_tiles, stream)
                 : go<VOID_DT_F16, false>(grad_c, ldg, b, ldb, block_rows, block_cols, n_blocks, M, N, K, grad_tiles, stream);
    default:
      return void_internal_fail(VOID_ERR_UNSUPPORTED, "gradient tiles are f32, bf16 or f16");
  }
}
