// void_format.hip — gfx950 kernels that build the VOID tile format from a
// CSR matrix on the device (csr_to_void, void/format.py:248-349), declared in
// include/void_amd.h.
//
// The reference walks every stored entry in a Python loop.  Here the same
// result comes from a few passes over device arrays:
//  1. mark:   one wave per CSR row sets a byte flag for every 32x32 block that
//             holds a stored entry (explicit zeros included);
//  2. rank:   blocks are visited in Morton order (the order the reference
//             sorts tiles into): code -> (block_row, block_col) by bit
//             de-interleaving; each flagged block gets its Morton rank in a
//             rank grid [n_block_rows][n_block_cols], and the block total is
//             written for the caller.  Grids of at most kSmallCodes codes use
//             one workgroup for the whole count / scan / rank; larger ones
//             count per chunk, scan the chunk counts, then rank;
//  3. emit:   one pass over the block grid writes block_rows, block_cols and
//             the Morton code of every flagged block at its rank and zeroes
//             its tile;
//  4. scatter: each stored entry is written into its tile (one wave per CSR
//             row again), four adjacent columns as one 16-byte store.
// Steps 1-2 run in void_csr_count_blocks (the caller then sizes the
// outputs from the block total); steps 3-4 in void_csr_to_tiles.  Inputs
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
constexpr int64_t kEmitGrid = 2048;  // emit: workgroups striding over the block grid
constexpr int kSmallThreads = 1024;                    // one-workgroup rank: threads
constexpr int kSmallPer = 32;                          // ... codes per thread
constexpr int64_t kSmallCodes = (int64_t)kSmallThreads * kSmallPer;  // ... the largest code space it takes
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

// Inverse of compact_even: the low 32 bits of x at the even positions.
__device__ __forceinline__ uint64_t spread_even(uint32_t v) {
  uint64_t x = v;
  x = (x | (x << 16)) & 0x0000ffff0000ffffull;
  x = (x | (x << 8)) & 0x00ff00ff00ff00ffull;
  x = (x | (x << 4)) & 0x0f0f0f0f0f0f0f0full;
  x = (x | (x << 2)) & 0x3333333333333333ull;
  x = (x | (x << 1)) & 0x5555555555555555ull;
  return x;
}

// Streaming (nontemporal) 16-byte accesses: data touched once per pass.
typedef int nt_v4i __attribute__((ext_vector_type(4)));
typedef float nt_v4f __attribute__((ext_vector_type(4)));
__device__ __forceinline__ int4 load_nt(const int32_t* p) {
  const nt_v4i v = __builtin_nontemporal_load(reinterpret_cast<const nt_v4i*>(p));
  return int4{v.x, v.y, v.z, v.w};
}
__device__ __forceinline__ float4 load_nt(const float* p) {
  const nt_v4f v = __builtin_nontemporal_load(reinterpret_cast<const nt_v4f*>(p));
  return float4{v.x, v.y, v.z, v.w};
}
__device__ __forceinline__ void store_nt(float* p, float4 v) {
  __builtin_nontemporal_store(nt_v4f{v.x, v.y, v.z, v.w}, reinterpret_cast<nt_v4f*>(p));
}

__global__ __launch_bounds__(kThreads) void fill_u8(uint8_t* p, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kThreads) p[i] = 0;
}

// 1. One wave per CSR row: flag the blocks of its entries.  Entries of a
// canonical row ascend, so a lane's four entries store one flag per distinct
// block, and the next group's indices are loaded before this one is used.
__global__ __launch_bounds__(kThreads) void mark_blocks(const int32_t* __restrict__ indptr,
                                                        const int32_t* __restrict__ indices, int32_t M,
                                                        int32_t n_bc, uint8_t* __restrict__ flags) {
  const int32_t r = blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
  if (r >= M) return;
  const int lane = threadIdx.x & 63;
  uint8_t* row_flags = flags + (int64_t)(r / kT) * n_bc;
  const int32_t b = indptr[r], e = indptr[r + 1];
  const int32_t head_end = min(e, (b + 3) & ~3);
  for (int32_t j = b + lane; j < head_end; j += 64) row_flags[indices[j] / kT] = 1;
  const int32_t body_end = head_end + ((e - head_end) & ~3);
  int32_t j = head_end + 4 * lane;
  if (j < body_end) {
    int4 c = load_nt(indices + j);
    while (true) {
      const int32_t jn = j + 256;
      const bool more = jn < body_end;
      int4 cn = c;
      if (more) cn = load_nt(indices + jn);
      const int32_t k0 = c.x / kT, k1 = c.y / kT, k2 = c.z / kT, k3 = c.w / kT;
      row_flags[k0] = 1;
      if (k1 != k0) row_flags[k1] = 1;
      if (k2 != k1) row_flags[k2] = 1;
      if (k3 != k2) row_flags[k3] = 1;
      if (!more) break;
      c = cn;
      j = jn;
    }
  }
  for (int32_t t = body_end + lane; t < e; t += 64) row_flags[indices[t] / kT] = 1;
}

// Even bits of a small x (below 64), packed: the row part of a low Morton
// code; constant-folded where x is.
__device__ __forceinline__ int even_bits6(int x) { return (x & 1) | ((x >> 1) & 2) | ((x >> 2) & 4); }

// Flags of the P codes [c0, c0 + P) into bit i of the result, all loads issued
// before any is used (codes outside the grid read flag 0 and count as 0).
// c0 is a multiple of P (a power of two), so code c0 + i has the block row
// and column of c0 plus those of i, which are constants once unrolled.
template <int P>
__device__ __forceinline__ uint32_t flag_bits(const uint8_t* flags, const Geometry& g, int64_t c0) {
  static_assert(P <= 32 && (P & (P - 1)) == 0, "one bit per code, aligned runs");
  const int32_t br0 = (int32_t)compact_even((uint64_t)c0), bc0 = (int32_t)compact_even((uint64_t)c0 >> 1);
  uint8_t f[P];
#pragma unroll
  for (int i = 0; i < P; ++i) {
    const int32_t br = br0 + even_bits6(i), bc = bc0 + even_bits6(i >> 1);
    const bool in = c0 + i < g.n_codes && br < g.n_br && bc < g.n_bc;
    f[i] = flags[in ? (int64_t)br * g.n_bc + bc : 0] & (in ? 1 : 0);
  }
  uint32_t m = 0;
#pragma unroll
  for (int i = 0; i < P; ++i) m |= (uint32_t)(f[i] != 0) << i;
  return m;
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
  const int n = __builtin_popcount(flag_bits<kPerThread>(flags, g, c0));
  const int incl = block_sum(n, sh);
  if (threadIdx.x == kThreads - 1) chunk[blockIdx.x] = incl;
}

// 3. One workgroup: chunk counts -> exclusive offsets, and the total (into
// the workspace and the caller's count).
__global__ __launch_bounds__(kThreads) void scan_chunks(int64_t n_chunks, int64_t* __restrict__ chunk,
                                                        int64_t* __restrict__ total, int64_t* __restrict__ count) {
  __shared__ int64_t sh[kThreads / 64 + 1];
  const int64_t per = (n_chunks + kThreads - 1) / kThreads;
  const int64_t b = (int64_t)threadIdx.x * per;
  int64_t s = 0;
  for (int64_t i = b; i < b + per && i < n_chunks; ++i) s += chunk[i];
  // Inclusive scan of s across the workgroup (wave shuffles, then wave sums).
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int64_t v = s;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int64_t o = __shfl_up(v, off, 64);
    if (lane >= off) v += o;
  }
  if (lane == 63) sh[wave] = v;
  __syncthreads();
  int64_t base = 0, all = 0;
#pragma unroll
  for (int w = 0; w < kThreads / 64; ++w) {
    if (w < wave) base += sh[w];
    all += sh[w];
  }
  int64_t run = base + v - s;
  for (int64_t i = b; i < b + per && i < n_chunks; ++i) {
    const int64_t c = chunk[i];
    chunk[i] = run;
    run += c;
  }
  if (threadIdx.x == 0) {
    *total = all;
    *count = all;
  }
}

// 2'. Small code spaces (at most kSmallCodes): count, scan and rank in one
// workgroup.  Thread t takes the contiguous codes [t kSmallPer, (t + 1) kSmallPer).
__global__ __launch_bounds__(kSmallThreads) void rank_small(Geometry g, const uint8_t* __restrict__ flags,
                                                            int32_t* __restrict__ rank, int64_t* __restrict__ total,
                                                            int64_t* __restrict__ count) {
  __shared__ int sh[kSmallThreads / 64];
  // The whole flag grid (n_br n_bc <= kSmallCodes bytes) in LDS, read with
  // coalesced 16-byte loads: the Morton walk then gathers from LDS.
  __shared__ __attribute__((aligned(16))) uint8_t lflags[kSmallCodes];
  const int64_t nb = (int64_t)g.n_br * g.n_bc;
  for (int64_t i = (int64_t)threadIdx.x * 16; i < nb; i += kSmallThreads * 16) {
    if (i + 16 <= nb) *reinterpret_cast<int4*>(lflags + i) = *reinterpret_cast<const int4*>(flags + i);
    else for (int64_t k = i; k < nb; ++k) lflags[k] = flags[k];
  }
  __syncthreads();
  const int64_t c0 = (int64_t)threadIdx.x * kSmallPer;
  const uint32_t bits = flag_bits<kSmallPer>(lflags, g, c0);
  const int32_t br0 = (int32_t)compact_even((uint64_t)c0), bc0 = (int32_t)compact_even((uint64_t)c0 >> 1);
  const int n = __builtin_popcount(bits);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int v = n;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int o = __shfl_up(v, off, 64);
    if (lane >= off) v += o;
  }
  if (lane == 63) sh[wave] = v;
  __syncthreads();
  int base = 0, all = 0;
#pragma unroll
  for (int w = 0; w < kSmallThreads / 64; ++w) {
    if (w < wave) base += sh[w];
    all += sh[w];
  }
  int pos = base + v - n;
  for (uint32_t m = bits; m; m &= m - 1) {
    const int k = __builtin_ctz(m);  // code c0 + k: c0's row and column plus k's
    const int32_t br = br0 + even_bits6(k), bc = bc0 + even_bits6(k >> 1);
    rank[(int64_t)br * g.n_bc + bc] = pos++;
  }
  if (threadIdx.x == 0) {
    *total = all;
    *count = all;
  }
}

// 2''. Large code spaces: the Morton rank of every flagged block from the
// chunk offsets.  LOCAL (at most kThreads chunks): chunk[] holds the counts,
// each workgroup sums those of the chunks below its own, and the last one
// writes the total, so no separate scan runs; otherwise chunk[] holds the
// offsets from scan_chunks.
template <bool LOCAL>
__global__ __launch_bounds__(kThreads) void rank_blocks(Geometry g, const uint8_t* __restrict__ flags,
                                                        const int64_t* __restrict__ chunk,
                                                        int32_t* __restrict__ rank, int64_t* __restrict__ total,
                                                        int64_t* __restrict__ count) {
  __shared__ int sh[kThreads / 64];
  __shared__ int s_base;
  const int64_t c0 = (int64_t)blockIdx.x * kChunk + (int64_t)threadIdx.x * kPerThread;
  const uint32_t bits = flag_bits<kPerThread>(flags, g, c0);
  const int32_t br0 = (int32_t)compact_even((uint64_t)c0), bc0 = (int32_t)compact_even((uint64_t)c0 >> 1);
  int64_t base;
  if constexpr (LOCAL) {
    // A chunk holds at most kChunk blocks, so the sums fit an int.
    const int below = threadIdx.x < blockIdx.x ? (int)chunk[threadIdx.x] : 0;
    const int b_incl = block_sum(below, sh);
    if (threadIdx.x == kThreads - 1) s_base = b_incl;
    __syncthreads();
    base = s_base;
  } else {
    base = chunk[blockIdx.x];
  }
  const int n = __builtin_popcount(bits);
  const int incl = block_sum(n, sh);
  if constexpr (LOCAL) {
    if (blockIdx.x == gridDim.x - 1 && threadIdx.x == kThreads - 1) {
      *total = base + incl;
      *count = base + incl;
    }
  }
  int64_t pos = base + (incl - n);
  for (uint32_t m = bits; m; m &= m - 1) {
    const int k = __builtin_ctz(m);  // code c0 + k: c0's row and column plus k's
    const int32_t br = br0 + even_bits6(k), bc = bc0 + even_bits6(k >> 1);
    rank[(int64_t)br * g.n_bc + bc] = (int32_t)pos++;
  }
}

// 3. A workgroup per flagged block (grid-stride over the block grid): its
// row, column and Morton code at its rank, and its zeroed tile (one 16-byte
// store per thread).  kEmitGrid workgroups: one per block would be bound by
// workgroup dispatch; staging runs of blocks per workgroup measured slower.
__global__ __launch_bounds__(kThreads) void emit_blocks(Geometry g, const uint8_t* __restrict__ flags,
                                                        const int32_t* __restrict__ rank,
                                                        int32_t* __restrict__ block_rows,
                                                        int32_t* __restrict__ block_cols,
                                                        int64_t* __restrict__ morton, float* __restrict__ values) {
  static_assert(kThreads * 4 == kT * kT, "one float4 per thread zeroes a tile");
  const int64_t nb = (int64_t)g.n_br * g.n_bc;
  for (int64_t blk = blockIdx.x; blk < nb; blk += gridDim.x) {
    if (!flags[blk]) continue;
    const int64_t pos = rank[blk];
    if (threadIdx.x == 0) {
      const int32_t br = (int32_t)(blk / g.n_bc), bc = (int32_t)(blk % g.n_bc);
      block_rows[pos] = br;
      block_cols[pos] = bc;
      morton[pos] = (int64_t)(spread_even((uint32_t)br) | (spread_even((uint32_t)bc) << 1));
    }
    store_nt(values + pos * (kT * kT) + 4 * threadIdx.x, float4{0.f, 0.f, 0.f, 0.f});
  }
}

// 4. One wave per CSR row: entries into their tiles.  Four entries of a
// lane at columns 4m .. 4m + 3 (one block, 16-byte aligned in the tile row)
// go out as one 16-byte store.
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
  auto put = [&](int32_t c, float v) { values[(int64_t)row_rank[c / kT] * (kT * kT) + rr * kT + (c % kT)] = v; };
  const int32_t b = indptr[r], e = indptr[r + 1];
  const int32_t head_end = min(e, (b + 3) & ~3);
  for (int32_t j = b + lane; j < head_end; j += 64) put(indices[j], data[j]);
  const int32_t body_end = head_end + ((e - head_end) & ~3);
  for (int32_t j = head_end + 4 * lane; j < body_end; j += 256) {
    const int4 c = load_nt(indices + j);
    const float4 v = load_nt(data + j);
    if ((c.x & 3) == 0 && c.w == c.x + 3) {
      store_nt(values + (int64_t)row_rank[c.x / kT] * (kT * kT) + rr * kT + (c.x % kT), v);
    } else {
      put(c.x, v.x);
      put(c.y, v.y);
      put(c.z, v.z);
      put(c.w, v.w);
    }
  }
  for (int32_t j = body_end + lane; j < e; j += 64) put(indices[j], data[j]);
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
  if (g.n_codes <= kSmallCodes) {
    hipLaunchKernelGGL(rank_small, dim3(1), dim3(kSmallThreads), 0, stream, g, w.flags, w.rank, w.total, n_blocks);
  } else {
    hipLaunchKernelGGL(count_chunks, dim3((unsigned)g.n_chunks), dim3(kThreads), 0, stream, g, w.flags, w.chunk);
    if (g.n_chunks <= kThreads) {
      hipLaunchKernelGGL(rank_blocks<true>, dim3((unsigned)g.n_chunks), dim3(kThreads), 0, stream, g, w.flags,
                         w.chunk, w.rank, w.total, n_blocks);
    } else {
      hipLaunchKernelGGL(scan_chunks, dim3(1), dim3(kThreads), 0, stream, g.n_chunks, w.chunk, w.total, n_blocks);
      hipLaunchKernelGGL(rank_blocks<false>, dim3((unsigned)g.n_chunks), dim3(kThreads), 0, stream, g, w.flags,
                         w.chunk, w.rank, nullptr, nullptr);
    }
  }
  return launched();
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
  if ((uintptr_t)values % 16) return void_internal_fail(VOID_ERR_ARG, "values must be 16-byte aligned");
  const Ws w = carve(workspace, g);
  const int64_t nb = (int64_t)g.n_br * g.n_bc;
  hipLaunchKernelGGL(emit_blocks, dim3((unsigned)(nb < kEmitGrid ? nb : kEmitGrid)), dim3(kThreads), 0, stream, g, w.flags,
                     w.rank, block_rows, block_cols, morton, values);
  hipLaunchKernelGGL(scatter_entries, dim3((M + 3) / 4), dim3(kThreads), 0, stream, indptr, indices, data, M, g.n_bc,
                     w.rank, values);
  return launched();
}

}  // extern "C"
