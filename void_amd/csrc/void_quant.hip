// void_quant.hip — gfx950 kernels for the quantisers on the SpMM path's
// input side: per-tile symmetric INT8 (quantize_void_tensor) and per-tile
// E4M3 (void_tensor_to_fp8), declared in include/void_amd.h.
//
// One wave64 per 32x32 fp32 tile: load q (0..3) of lane l reads values
// 256 q + 4 l .. + 3, so each load instruction reads 1 KB contiguously and
// requests every cache line once; the wave reduces the tile's amax with
// cross-lane max, and store q writes the lane's 4 codes of those values (256
// contiguous bytes per instruction).  The work is HBM-bound byte traffic:
// 4 KB in, 1 KB + 4 bytes out per tile.  Rounding follows the reference's torch arithmetic
// exactly: IEEE fp32 division and multiplication, round half to even.

#include <hip/hip_runtime.h>

#include <algorithm>

#include <cstdint>

#include "void_amd.h"

extern "C" __attribute__((visibility("hidden"))) int void_internal_fail(int code, const char* msg);

namespace {

constexpr int kTileElems = 32 * 32;
constexpr int kWavesPerBlock = 4;

typedef float v4f __attribute__((ext_vector_type(4)));
typedef int v4i __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

// Loads this lane's 16 values of tile t (x[4 q + i] = value 256 q + 4 lane +
// i) and returns the tile's amax (max |x|, which equals max(|min|, |max|) for
// finite values).
__device__ __forceinline__ float load_tile(const float* tiles, int64_t t, int lane, float (&x)[16]) {
  const v4f* p = reinterpret_cast<const v4f*>(tiles + t * kTileElems) + lane;
  float m = 0.f;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const v4f v = __builtin_nontemporal_load(p + 64 * q);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[4 * q + i] = v[i];
      m = fmaxf(m, fabsf(v[i]));
    }
  }
  return wave_max(m);
}

__device__ __forceinline__ uint32_t pack4(int a, int b, int c, int d) {
  return (uint32_t)(a & 0xff) | ((uint32_t)(b & 0xff) << 8) | ((uint32_t)(c & 0xff) << 16) |
         ((uint32_t)(d & 0xff) << 24);
}

// Codes of this lane's 16 values (the layout of load_tile) into the tile's
// 1 KB of codes: store w writes values 256 w + 4 lane .. + 3.
template <class C>
__device__ __forceinline__ void store_codes(void* dst, int lane, const C (&c)[16]) {
  uint32_t* d = reinterpret_cast<uint32_t*>(dst) + lane;
#pragma unroll
  for (int w = 0; w < 4; ++w)
    __builtin_nontemporal_store(pack4((int)c[4 * w], (int)c[4 * w + 1], (int)c[4 * w + 2], (int)c[4 * w + 3]),
                                d + 64 * w);
}

// int_quant.py:178-214 (symmetric min/max scale), :254-305 (quantize_tensor):
// s = max(amax / 128, 1e-8); q = clamp(round_half_even(x / s), -128, 127).
__global__ __launch_bounds__(64 * kWavesPerBlock) void quantize_i8_kernel(const float* __restrict__ tiles,
                                                                          int n_tiles, int8_t* __restrict__ q,
                                                                          float* __restrict__ scales) {
  const int lane = threadIdx.x & 63;
  const int64_t t = (int64_t)blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6);
  if (t >= n_tiles) return;
  float x[16];
  const float amax = load_tile(tiles, t, lane, x);
  const float s = fmaxf(__fdiv_rn(amax, 128.0f), 1e-8f);
  int c[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) c[i] = (int)fminf(fmaxf(rintf(__fdiv_rn(x[i], s)), -128.0f), 127.0f);
  store_codes(q + t * kTileElems, lane, c);
  if (lane == 0) scales[t] = s;
}

// E4M3FN code of a finite float32 in [-448, 448], round to nearest even.
// Normal range (|x| >= 2^-6): keep 3 mantissa bits with RNE on the fp32
// mantissa; a carry out of the mantissa bumps the exponent.  Subnormal range:
// the code is round_half_even(|x| * 2^9) (exact scaling by a power of two),
// which also yields the smallest normal (code 8) when it rounds up to 2^-6.
__device__ __forceinline__ uint32_t e4m3_code(float x) {
  const uint32_t u = __float_as_uint(x);
  const uint32_t sign = (u >> 24) & 0x80u;
  const float a = fabsf(x);
  uint32_t code;
  if (a < 0.015625f) {
    code = (uint32_t)rintf(a * 512.0f);
  } else {
    const uint32_t ua = u & 0x7fffffffu;
    const int e = (int)(ua >> 23) - 127;  // -6 .. 8
    const uint32_t m = ua & 0x7fffffu;
    uint32_t m3 = (m + 0x7ffffu + ((m >> 20) & 1u)) >> 20;  // RNE to 3 bits, may reach 8
    int ee = e + 7;
    if (m3 == 8u) {
      m3 = 0u;
      ee += 1;
    }
    code = ((uint32_t)ee << 3) | m3;
  }
  return sign | code;
}

// fp8.py:81-105 (first-call scale from a zero amax history: amax / 448,
// clamp 1e-12), :185-229 (x * (1 / scale), clamp to +-448, cast to E4M3FN).
__global__ __launch_bounds__(64 * kWavesPerBlock) void quantize_fp8_kernel(const float* __restrict__ tiles,
                                                                           int n_tiles, uint8_t* __restrict__ q,
                                                                           float* __restrict__ scales,
                                                                           float* __restrict__ amaxes) {
  const int lane = threadIdx.x & 63;
  const int64_t t = (int64_t)blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6);
  if (t >= n_tiles) return;
  float x[16];
  const float amax = load_tile(tiles, t, lane, x);
  const float s = fmaxf(__fdiv_rn(amax, 448.0f), 1e-12f);
  const float inv = __fdiv_rn(1.0f, s);
  uint32_t c[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) c[i] = e4m3_code(fminf(fmaxf(__fmul_rn(x[i], inv), -448.0f), 448.0f));
  store_codes(q + t * kTileElems, lane, c);
  if (lane == 0) {
    scales[t] = s;
    if (amaxes) amaxes[t] = amax;
  }
}

int check_args(const float* tiles, int32_t n_tiles, const void* q, const float* scales) {
  if (n_tiles < 0) return void_internal_fail(VOID_ERR_ARG, "negative tile count");
  if (n_tiles == 0) return VOID_OK;
  if (!tiles || !q || !scales) return void_internal_fail(VOID_ERR_ARG, "null tile, code or scale pointer");
  if ((uintptr_t)tiles % 16 || (uintptr_t)q % 16)
    return void_internal_fail(VOID_ERR_ARG, "tiles and codes must be 16-byte aligned");
  return 1;
}

// Per-tensor symmetric INT8 quantisation of a float B (int_quant.py:178-214,
// 308-325 with qmin = -128, qmax = 127): scale = max(max |b| / 128, 1e-8),
// q = clamp(rint(b / scale), -128, 127) with IEEE division.  Two launches:
// the first writes one partial max |b| per workgroup (as bits: for the
// non-negative floats the integer order is the float order, and a NaN's
// bits exceed infinity's), the second reduces the partials in every
// workgroup, quantises its share and has workgroup 0 write the scale.
constexpr int kQbThreads = 256;
constexpr int kQbMaxPartials = 1024;

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = max(v, (uint32_t)__shfl_xor((int)v, o, 64));
  return v;
}

__device__ __forceinline__ uint32_t block_max_u32(uint32_t v, uint32_t* red) {
  v = wave_max_u32(v);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  uint32_t m = red[0];
#pragma unroll
  for (int w = 1; w < kQbThreads / 64; ++w) m = max(m, red[w]);
  return m;
}

__global__ __launch_bounds__(kQbThreads) void b_amax_kernel(const float* __restrict__ b, int64_t n,
                                                          uint32_t* __restrict__ partials) {
  __shared__ uint32_t red[kQbThreads / 64];
  typedef float v4f __attribute__((ext_vector_type(4)));
  uint32_t m = 0;
  const int64_t n4 = n / 4;
  for (int64_t i = (int64_t)blockIdx.x * kQbThreads + threadIdx.x; i < n4; i += (int64_t)gridDim.x * kQbThreads) {
    const v4f x = __builtin_nontemporal_load(reinterpret_cast<const v4f*>(b) + i);
#pragma unroll
    for (int k = 0; k < 4; ++k) m = max(m, __float_as_uint(x[k]) & 0x7fffffffu);
  }
  for (int64_t i = 4 * n4 + (int64_t)blockIdx.x * kQbThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kQbThreads)
    m = max(m, __float_as_uint(b[i]) & 0x7fffffffu);
  m = block_max_u32(m, red);
  if (threadIdx.x == 0) partials[blockIdx.x] = m;
}

__global__ __launch_bounds__(kQbThreads) void b_quant_kernel(const float* __restrict__ b, int64_t n,
                                                           const uint32_t* __restrict__ partials, int32_t n_partials,
                                                           int8_t* __restrict__ q, float* __restrict__ scale_out) {
  __shared__ uint32_t red[kQbThreads / 64];
  typedef float v4f __attribute__((ext_vector_type(4)));
  uint32_t m = 0;
  for (int i = threadIdx.x; i < n_partials; i += kQbThreads) m = max(m, partials[i]);
  m = block_max_u32(m, red);
  // torch.clamp(scale, min=1e-8) keeps a NaN scale (fmaxf would drop it).
  const float amax = __uint_as_float(m) / 128.0f;
  const float scale = amax != amax ? amax : fmaxf(amax, 1e-8f);
  if (blockIdx.x == 0 && threadIdx.x == 0) scale_out[0] = scale;
  auto code = [&](float x) -> uint32_t {
    const float r = __builtin_rintf(__fdiv_rn(x, scale));
    return (uint32_t)(uint8_t)(int8_t)(int)fminf(fmaxf(r, -128.0f), 127.0f);
  };
  const int64_t n4 = n / 4;
  for (int64_t i = (int64_t)blockIdx.x * kQbThreads + threadIdx.x; i < n4; i += (int64_t)gridDim.x * kQbThreads) {
    const v4f x = __builtin_nontemporal_load(reinterpret_cast<const v4f*>(b) + i);
    const uint32_t w = code(x[0]) | (code(x[1]) << 8) | (code(x[2]) << 16) | (code(x[3]) << 24);
    reinterpret_cast<uint32_t*>(q)[i] = w;
  }
  for (int64_t i = 4 * n4 + (int64_t)blockIdx.x * kQbThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kQbThreads)
    q[i] = (int8_t)code(b[i]);
}

// dst[c][r] = src[r][c] for a rows x cols byte matrix (int8 or E4M3 codes):
// a column-major B made row-major for the SpMM's LDS-DMA ring.  A workgroup
// moves a 64-row x 256-column tile through LDS: 16-byte loads along the
// source rows, then 16-byte stores along the destination rows, each built
// from 16 bytes of one LDS column.  rows and cols are multiples of 16.
constexpr int kTRows = 64, kTCols = 256, kTPad = 16;

__global__ __launch_bounds__(256) void transpose_b8_kernel(const uint8_t* __restrict__ src, int64_t ld_src,
                                                          int32_t rows, int32_t cols, uint8_t* __restrict__ dst,
                                                          int64_t ld_dst) {
  __shared__ __attribute__((aligned(16))) uint8_t t[kTRows][kTCols + kTPad];
  typedef int v4i __attribute__((ext_vector_type(4)));
  const int r0 = blockIdx.y * kTRows, c0 = blockIdx.x * kTCols;
  const int tid = threadIdx.x;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int q = tid + 256 * i, r = q >> 4, ch = q & 15;
    v4i v = v4i{0, 0, 0, 0};
    if (r0 + r < rows && c0 + 16 * ch < cols)
      v = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(src + (int64_t)(r0 + r) * ld_src + c0 + 16 * ch));
    *reinterpret_cast<v4i*>(&t[r][16 * ch]) = v;
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int q = tid + 256 * i, c = q >> 2, rc = q & 3;
    if (c0 + c < cols && r0 + 16 * rc < rows) {
      uint32_t w[4];
#pragma unroll
      for (int k = 0; k < 4; ++k)
        w[k] = (uint32_t)t[16 * rc + 4 * k][c] | ((uint32_t)t[16 * rc + 4 * k + 1][c] << 8) |
               ((uint32_t)t[16 * rc + 4 * k + 2][c] << 16) | ((uint32_t)t[16 * rc + 4 * k + 3][c] << 24);
      *reinterpret_cast<v4i*>(dst + (int64_t)(c0 + c) * ld_dst + r0 + 16 * rc) =
          v4i{(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
    }
  }
}

}  // namespace

extern "C" {

int void_quantize_b_i8(const float* b, int64_t n, int8_t* q, float* scale, uint32_t* partials,
                       hipStream_t stream) {
  void_internal_fail(VOID_OK, "");
  if (n < 0) return void_internal_fail(VOID_ERR_ARG, "negative size");
  if (n == 0) return VOID_OK;
  if (!b || !q || !scale || !partials) return void_internal_fail(VOID_ERR_ARG, "null pointer");
  if ((uintptr_t)b % 16 || (uintptr_t)q % 4) return void_internal_fail(VOID_ERR_ARG, "b must be 16-byte, q 4-byte aligned");
  const int g = (int)std::min<int64_t>(kQbMaxPartials, std::max<int64_t>(1, (n + 4095) / 4096));
  hipLaunchKernelGGL(b_amax_kernel, dim3(g), dim3(kQbThreads), 0, stream, b, n, partials);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return void_internal_fail(VOID_ERR_HIP, hipGetErrorString(e));
  const int gq = (int)std::min<int64_t>(2048, std::max<int64_t>(1, (n + 4095) / 4096));
  hipLaunchKernelGGL(b_quant_kernel, dim3(gq), dim3(kQbThreads), 0, stream, b, n, partials, g, q, scale);
  e = hipGetLastError();
  if (e != hipSuccess) return void_internal_fail(VOID_ERR_HIP, hipGetErrorString(e));
  return VOID_OK;
}

int void_transpose_b8(const void* src, int64_t ld_src, int32_t rows, int32_t cols, void* dst, int64_t ld_dst,
                      hipStream_t stream) {
  void_internal_fail(VOID_OK, "");
  if (rows < 0 || cols < 0) return void_internal_fail(VOID_ERR_ARG, "negative size");
  if ((int64_t)rows * cols == 0) return VOID_OK;
  if (!src || !dst) return void_internal_fail(VOID_ERR_ARG, "null pointer");
  if (rows % 16 || cols % 16 || ld_src < cols || ld_dst < rows || ld_src % 16 || ld_dst % 16 ||
      ((uintptr_t)src | (uintptr_t)dst) % 16)
    return void_internal_fail(VOID_ERR_UNSUPPORTED,
                              "void_transpose_b8 needs rows, cols and leading dimensions multiples of 16 and "
                              "16-byte aligned arrays");
  const dim3 grid((cols + kTCols - 1) / kTCols, (rows + kTRows - 1) / kTRows);
  if (grid.y > 65535) return void_internal_fail(VOID_ERR_ARG, "too many rows");
  hipLaunchKernelGGL(transpose_b8_kernel, grid, dim3(256), 0, stream, static_cast<const uint8_t*>(src), ld_src, rows,
                     cols, static_cast<uint8_t*>(dst), ld_dst);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return void_internal_fail(VOID_ERR_HIP, hipGetErrorString(e));
  return VOID_OK;
}

int void_quantize_tiles_i8(const float* tiles, int32_t n_tiles, int8_t* q, float* scales, hipStream_t stream) {
  void_internal_fail(VOID_OK, "");
  const int st = check_args(tiles, n_tiles, q, scales);
  if (st <= 0) return st;
  const int grid = (n_tiles + kWavesPerBlock - 1) / kWavesPerBlock;
  hipLaunchKernelGGL(quantize_i8_kernel, dim3(grid), dim3(64 * kWavesPerBlock), 0, stream, tiles, n_tiles, q,
                     scales);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return void_internal_fail(VOID_ERR_HIP, hipGetErrorString(e));
  return VOID_OK;
}

int void_quantize_tiles_fp8(const float* tiles, int32_t n_tiles, uint8_t* q, float* scales, float* amax,
                            hipStream_t stream) {
  void_internal_fail(VOID_OK, "");
  const int st = check_args(tiles, n_tiles, q, scales);
  if (st <= 0) return st;
  const int grid = (n_tiles + kWavesPerBlock - 1) / kWavesPerBlock;
  hipLaunchKernelGGL(quantize_fp8_kernel, dim3(grid), dim3(64 * kWavesPerBlock), 0, stream, tiles, n_tiles, q,
                     scales, amax);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return void_internal_fail(VOID_ERR_HIP, hipGetErrorString(e));
  return VOID_OK;
}

}  // extern "C"
