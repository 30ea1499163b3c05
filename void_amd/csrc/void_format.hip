// void_format.hip — gfx950 kernels that build the VOID tile format from a
// CSR matrix on the device (csr_to_void, void/format.py:248-349), declared in
// include/void_amd.h.
//
// The reference walks every stored entry in a Python loop.  Here the same
// result comes from four passes over device arrays:
//  1. mark:   one wave per CSR row sets a byte flag for every 32x32 block that
//             holds a stored entry (explicit zeros included);
//  2. count:  blocks are visited in Morton order (the order the reference
//             sorts tiles into): code -> (block_row, block_col) by bit
//             de-interleaving, 4096 codes per workgroup, flags counted;
//  3. scan:   one workgroup turns the per-chunk counts into offsets and the
//             block total;
//  4. rank:   every flagged block gets its Morton rank; block_rows,
//             block_cols and morton codes are written at that rank, and a
//             rank grid [n_block_rows][n_block_cols] is kept for
//  5. scatter: tiles are zeroed, then each stored entry is written into its
//             tile (one wave per CSR row again).
// Steps 1-3 run in void_csr_count_blocks (the caller then sizes the
// outputs from the block total); steps 4-5 in void_csr_to_tiles.  Inputs
// must be canonical CSR (no duplicate entries): with duplicates the
// reference keeps the last one, an order a parallel scatter does not have.

#include <hip/hip_runtime.h>

#include <cstdint>

#include "void_amd.h"

extern "C" __attribute__((visibility("hidden"))) int void_internal_fail(int code, const char* msg);

namespace {

constexpr int kT = 32;
constexpr int kChunk = 4096;       // Morton codes per workgroup in count / rank
constexpr int kThreads = 256;
constexpr int kPerThread = kChunk / kThreads;
constexpr int64_t kMaxGrid = (int64_t)1 << 28;   // blocks in the block grid
constexpr int64_t kMaxCodes = (int64_t)1 << 30;  // Morton codes of the padded square grid

struct Geometry {
  int32_t n_br, n_bc;  // block grid
  int32_t log2p;       // side of the padded power-of-two square grid
  int64_t n_codes;     // (1 << log2p)^2
  int64_t n_chunks;    // ceil(n_codes / kChunk)
};

int geometry(int32_t M, int32_t N, Geometry& g) {
  g.n_br = (M + kT - 1) / kT;
  g.n_bc = (N + kT - 1) / kT;
  const int32_t side = g.n_br > g.n_bc ? g.n_br : g.n_bc;
  g.log2p = 0;
  while ((1 << g.log2p) < side) ++g.log2p;
  g.n_codes = (int64_t)1 << (2 * g.log2p);
  g.n_chunks = (g.n_codes + kChunk - 1) / kChunk;
  if ((int64_t)g.n_br * g.n_bc > kMaxGrid || g.n_codes > kMaxCodes) return VOID_ERR_UNSUPPORTED;
  return VOID_OK;
}

// Workspace: flags (bytes, one per block) | rank grid (int32 per block) |
// chunk counts (int64 per chunk, then offsets) | total (int64).
struct Ws {
  uint8_t* flags;
  int32_t* rank;
  int64_t* chunk;
  int64_t* total;
};

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

size_t ws_bytes(const Geometry& g) {
  const size_t nb = (size_t)g.n_br * g.n_bc;
  return align256(nb) + align256(nb * 4) + align256((size_t)g.n_chunks * 8) + 256;
}

Ws carve(void* base, const Geometry& g) {
  const size_t nb = (size_t)g.n_br * g.n_bc;
  uint8_t* p = static_cast<uint8_t*>(base);
  Ws w;
  w.flags = p;
  p += align256(nb);
  w.rank = reinterpret_cast<int32_t*>(p);
  p += align256(nb * 4);
  w.chunk = reinterpret_cast<int64_t*>(p);
  p += align256((size_t)g.n_chunks * 8);
  w.total = reinterpret_cast<int64_t*>(p);
  return w;
}

// Even bits of x packed into the low half (inverse of the interleave that
// puts row bits at even positions, format.py:41-51).
__device__ __forceinline__ uint32_t compact_even(uint64_t x) {
  x &= 0x5555555555555555ull;
  x = (x | (x >> 1)) & 0x3333333333333333ull;
  x = (x | (x >> 2)) & 0x0f0f0f0f0f0f0f0full;
  x = (x | (x >> 4)) & 0x00ff00ff00ff00ffull;
  x = (x | (x >> 8)) & 0x0000ffff0000ffffull;
  x = (x | (x >> 16)) & 0x00000000ffffffffull;
  return (uint32_t)x;
}

__global__ __launch_bounds__(kThreads) void fill_u8(uint8_t* p, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kThreads) p[i] = 0;
}

__global__ __launch_bounds__(kThreads) void fill_f32(float* p, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kThreads)
    p[i] = 0.f;
}

// Entries [b, e) of one CSR row, four per lane per step: the 16-byte-aligned
// middle with vector loads, the unaligned head and the tail one by one.
template <typename F>
__device__ __forceinline__ void for_row_entries(int32_t b, int32_t e, int lane, const int32_t* __restrict__ indices,
                                                const float* __restrict__ data, F&& f) {
  const int32_t head_end = min(e, (b + 3) & ~3);
  for (int32_t j = b + lane; j < head_end; j += 64) f(indices[j], data ? data[j] : 0.f);
  const int32_t body_end = head_end + ((e - head_end) & ~3);
  for (int32_t j = head_end + 4 * lane; j < body_end; j += 256) {
    const int4 c = *reinterpret_cast<const int4*>(indices + j);
    float4 v = {0.f, 0.f, 0.f, 0.f};
    if (data) v = *reinterpret_cast<const float4*>(data + j);
    f(c.x, v.x);
    f(c.y, v.y);
    f(c.z, v.z);
    f(c.w, v.w);
  }
  for (int32_t j = body_end + lane; j < e; j += 64) f(indices[j], data ? data[j] : 0.f);
}

// 1. One wave per CSR row: flag the blocks of its entries.
__global__ __launch_bounds__(kThreads) void mark_blocks(const int32_t* __restrict__ indptr,
                                                        const int32_t* __restrict__ indices, int32_t M,
                                                        int32_t n_bc, uint8_t* __restrict__ flags) {
  const int32_t r = blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
  if (r >= M) return;
  const int lane = threadIdx.x & 63;
  uint8_t* row_flags = flags + (int64_t)(r / kT) * n_bc;
  for_row_entries(indptr[r], indptr[r + 1], lane, indices, nullptr,
                  [&](int32_t c, float) { row_flags[c / kT] = 1; });
}

__device__ __forceinline__ bool flag_at(const uint8_t* flags, const Geometry& g, int64_t code, int32_t& br,
                                        int32_t& bc) {
  br = (int32_t)compact_even((uint64_t)code);
  bc = (int32_t)compact_even((uint64_t)code >> 1);
  return br < g.n_br && bc < g.n_bc && flags[(int64_t)br * g.n_bc + bc];
}

__device__ __forceinline__ int block_sum(int v, int* sh) {
  // inclusive scan across the workgroup; returns this thread's inclusive sum
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int o = __shfl_up(v, off, 64);
    if (lane >= off) v += o;
  }
  if (lane == 63) sh[wave] = v;
  __syncthreads();
  int base = 0;
  for (int w = 0; w < wave; ++w) base += sh[w];
  __syncthreads();
  return base + v;
}

// 2. Count flagged blocks per chunk of Morton codes.
__global__ __launch_bounds__(kThreads) void count_chunks(Geometry g, const uint8_t* __restrict__ flags,
                                                         int64_t* __restrict__ chunk) {
  __shared__ int sh[kThreads / 64];
  const int64_t c0 = (int64_t)blockIdx.x * kChunk + (int64_t)threadIdx.x * kPerThread;
  int n = 0;
  for (int i = 0; i < kPerThread; ++i) {
    int32_t br, bc;
    if (c0 + i < g.n_codes && flag_at(flags, g, c0 + i, br, bc)) ++n;
  }
  const int incl = block_sum(n, sh);
  if (threadIdx.x == kThreads - 1) chunk[blockIdx.x] = incl;
}

// 3. One workgroup: chunk counts -> exclusive offsets, and the total.
__global__ __launch_bounds__(kThreads) void scan_chunks(int64_t n_chunks, int64_t* __restrict__ chunk,
                                                        int64_t* __restrict__ total) {
  __shared__ int64_t sh[kThreads];
  const int64_t per = (n_chunks + kThreads - 1) / kThreads;
  const int64_t b = (int64_t)threadIdx.x * per;
  int64_t s = 0;
  for (int64_t i = b; i < b + per && i < n_chunks; ++i) s += chunk[i];
  sh[threadIdx.x] = s;
  __syncthreads();
  if (threadIdx.x == 0) {
    int64_t run = 0;
    for (int t = 0; t < kThreads; ++t) {
      const int64_t v = sh[t];
      sh[t] = run;
      run += v;
    }
    *total = run;
  }
  __syncthreads();
  int64_t run = sh[threadIdx.x];
  for (int64_t i = b; i < b + per && i < n_chunks; ++i) {
    const int64_t v = chunk[i];
    chunk[i] = run;
    run += v;
  }
}

// 4. Morton rank of every flagged block; per-tile metadata at that rank.
__global__ __launch_bounds__(kThreads) void rank_blocks(Geometry g, const uint8_t* __restrict__ flags,
                                                        const int64_t* __restrict__ chunk,
                                                        int32_t* __restrict__ rank, int32_t* __restrict__ block_rows,
                                                        int32_t* __restrict__ block_cols,
                                                        int64_t* __restrict__ morton) {
  __shared__ int sh[kThreads / 64];
  const int64_t c0 = (int64_t)blockIdx.x * kChunk + (int64_t)threadIdx.x * kPerThread;
  int n = 0;
  for (int i = 0; i < kPerThread; ++i) {
    int32_t br, bc;
    if (c0 + i < g.n_codes && flag_at(flags, g, c0 + i, br, bc)) ++n;
  }
  const int incl = block_sum(n, sh);
  int64_t pos = chunk[blockIdx.x] + (incl - n);
  for (int i = 0; i < kPerThread; ++i) {
    int32_t br, bc;
    if (c0 + i < g.n_codes && flag_at(flags, g, c0 + i, br, bc)) {
      rank[(int64_t)br * g.n_bc + bc] = (int32_t)pos;
      block_rows[pos] = br;
      block_cols[pos] = bc;
      morton[pos] = c0 + i;
      ++pos;
    }
  }
}

// 5. One wave per CSR row: entries into their tiles.
__global__ __launch_bounds__(kThreads) void scatter_entries(const int32_t* __restrict__ indptr,
                                                            const int32_t* __restrict__ indices,
                                                            const float* __restrict__ data, int32_t M, int32_t n_bc,
                                                            const int32_t* __restrict__ rank,
                                                            float* __restrict__ values) {
  const int32_t r = blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
  if (r >= M) return;
  const int lane = threadIdx.x & 63;
  const int32_t* row_rank = rank + (int64_t)(r / kT) * n_bc;
  const int rr = r % kT;
  for_row_entries(indptr[r], indptr[r + 1], lane, indices, data, [&](int32_t c, float v) {
    values[(int64_t)row_rank[c / kT] * (kT * kT) + rr * kT + (c % kT)] = v;
  });
}

int launched() {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return void_internal_fail(VOID_ERR_HIP, hipGetErrorString(e));
  return VOID_OK;
}

int grid_for(int64_t n) {
  const int64_t b = (n + kThreads - 1) / kThreads;
  return (int)(b < 65536 ? (b > 0 ? b : 1) : 65536);
}

}  // namespace

extern "C" {

size_t void_csr_workspace_bytes(int32_t M, int32_t N) {
  Geometry g;
  if (M < 0 || N < 0 || geometry(M, N, g) != VOID_OK) return 0;
  return ws_bytes(g);
}

int void_csr_count_blocks(const int32_t* indptr, const int32_t* indices, int32_t M, int32_t N, void* workspace,
                          size_t workspace_bytes, int64_t* n_blocks, hipStream_t stream) {
  void_internal_fail(VOID_OK, "");
  if (M < 0 || N < 0) return void_internal_fail(VOID_ERR_ARG, "negative matrix size");
  Geometry g;
  if (geometry(M, N, g) != VOID_OK)
    return void_internal_fail(VOID_ERR_UNSUPPORTED, "block grid too large for the device conversion");
  if (!indptr || !workspace || !n_blocks || (M > 0 && !indices))
    return void_internal_fail(VOID_ERR_ARG, "null indptr, indices, workspace or count pointer");
  if ((uintptr_t)indices % 16) return void_internal_fail(VOID_ERR_ARG, "indices must be 16-byte aligned");
  if (workspace_bytes < ws_bytes(g)) return void_internal_fail(VOID_ERR_WORKSPACE, "workspace too small");
  const Ws w = carve(workspace, g);
  const int64_t nb = (int64_t)g.n_br * g.n_bc;
  hipLaunchKernelGGL(fill_u8, dim3(grid_for(nb)), dim3(kThreads), 0, stream, w.flags, nb);
  if (M > 0)
    hipLaunchKernelGGL(mark_blocks, dim3((M + 3) / 4), dim3(kThreads), 0, stream, indptr, indices, M, g.n_bc,
                       w.flags);
  hipLaunchKernelGGL(count_chunks, dim3((unsigned)g.n_chunks), dim3(kThreads), 0, stream, g, w.flags, w.chunk);
  hipLaunchKernelGGL(scan_chunks, dim3(1), dim3(kThreads), 0, stream, g.n_chunks, w.chunk, w.total);
  int st = launched();
  if (st) return st;
  const hipError_t e = hipMemcpyAsync(n_blocks, w.total, sizeof(int64_t), hipMemcpyDeviceToDevice, stream);
  if (e != hipSuccess) return void_internal_fail(VOID_ERR_HIP, hipGetErrorString(e));
  return VOID_OK;
}

int void_csr_to_tiles(const int32_t* indptr, const int32_t* indices, const float* data, int32_t M, int32_t N,
                      void* workspace, size_t workspace_bytes, int64_t n_blocks, float* values,
                      int32_t* block_rows, int32_t* block_cols, int64_t* morton, hipStream_t stream) {
  void_internal_fail(VOID_OK, "");
  if (M < 0 || N < 0 || n_blocks < 0) return void_internal_fail(VOID_ERR_ARG, "negative size");
  Geometry g;
  if (geometry(M, N, g) != VOID_OK)
    return void_internal_fail(VOID_ERR_UNSUPPORTED, "block grid too large for the device conversion");
  if (n_blocks > (int64_t)g.n_br * g.n_bc) return void_internal_fail(VOID_ERR_ARG, "more blocks than the grid holds");
  if (n_blocks == 0) return VOID_OK;
  if (!indptr || !indices || !data || !workspace || !values || !block_rows || !block_cols || !morton)
    return void_internal_fail(VOID_ERR_ARG, "null pointer");
  if ((uintptr_t)indices % 16 || (uintptr_t)data % 16)
    return void_internal_fail(VOID_ERR_ARG, "indices and data must be 16-byte aligned");
  if (workspace_bytes < ws_bytes(g)) return void_internal_fail(VOID_ERR_WORKSPACE, "workspace too small");
  const Ws w = carve(workspace, g);
  hipLaunchKernelGGL(rank_blocks, dim3((unsigned)g.n_chunks), dim3(kThreads), 0, stream, g, w.flags, w.chunk,
                     w.rank, block_rows, block_cols, morton);
  const int64_t nv = n_blocks * kT * kT;
  hipLaunchKernelGGL(fill_f32, dim3(grid_for(nv / 4)), dim3(kThreads), 0, stream, values, nv);
  hipLaunchKernelGGL(scatter_entries, dim3((M + 3) / 4), dim3(kThreads), 0, stream, indptr, indices, data, M, g.n_bc,
                     w.rank, values);
  return launched();
}

}  // extern "C"
