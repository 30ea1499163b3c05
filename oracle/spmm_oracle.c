/*
 * spmm_oracle.c — CPU restatement of the reference's quantised block-sparse
 * SpMM arithmetic.  TEST INFRASTRUCTURE ONLY: used by tests/, by the smoke
 * check and by bench.py's cpu_baseline leg as the checker; never by the
 * product path.
 *
 * Tiles are given in block-row-major order: tiles of block-row r are
 * [row_ptr[r], row_ptr[r+1]) with ascending block column, tile t covering
 * A[32r .. 32r+31][32*col_idx[t] .. +31], row-major 32x32.  B is row-major
 * K x N with leading dimension ldb.
 *
 * Build with -ffp-contract=off: the fp32 epilogue must round every product
 * and every sum separately, as the reference's Triton code does.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define TILE 32

/* acc[m][n] = sum over the tiles of m's block-row of sum_k A_t[m%32][k] * B[32 col_t + k][n],
 * in exact integer arithmetic (int_quant.py:484-516, tl.dot int8 x int8 -> int32).
 * Returns 0, or -1 if a sum leaves the int32 range. */
int oracle_i8_acc(const int8_t* tiles, const int32_t* row_ptr, const int32_t* col_idx,
                  int32_t n_block_rows, int32_t M, int32_t K, const int8_t* b, int64_t ldb,
                  int32_t N, int32_t* acc, int64_t ldacc) {
  int bad = 0;
#pragma omp parallel for schedule(dynamic, 1) reduction(| : bad)
  for (int32_t r = 0; r < n_block_rows; ++r) {
    int64_t sum[TILE][1024];
    for (int32_t n0 = 0; n0 < N; n0 += 1024) {
      const int32_t nn = (N - n0) < 1024 ? (N - n0) : 1024;
      for (int i = 0; i < TILE; ++i) memset(sum[i], 0, sizeof(int64_t) * (size_t)nn);
      for (int32_t t = row_ptr[r]; t < row_ptr[r + 1]; ++t) {
        const int8_t* tile = tiles + (int64_t)t * TILE * TILE;
        for (int k = 0; k < TILE; ++k) {
          const int64_t kk = (int64_t)col_idx[t] * TILE + k;
          if (kk >= K) break;
          const int8_t* brow = b + kk * ldb + n0;
          for (int i = 0; i < TILE; ++i) {
            const int64_t av = tile[i * TILE + k];
            if (av == 0) continue;
            for (int32_t n = 0; n < nn; ++n) sum[i][n] += av * (int64_t)brow[n];
          }
        }
      }
      for (int i = 0; i < TILE; ++i) {
        const int64_t m = (int64_t)r * TILE + i;
        if (m >= M) break;
        for (int32_t n = 0; n < nn; ++n) {
          if (sum[i][n] > INT32_MAX || sum[i][n] < INT32_MIN) bad = 1;
          acc[m * ldacc + n0 + n] = (int32_t)sum[i][n];
        }
      }
    }
  }
  return bad ? -1 : 0;
}

/* Row-mean epilogue of void_spmm_int8_kernel (int_quant.py:519-526):
 *   S[n] = ((0 + fl(s_a[t0] * s_b[n])) + fl(s_a[t1] * s_b[n])) + ...   (fp32, tile order)
 *   out[m][n] = f32(acc[m][n]) * (S[n] / f32(n_tiles)), or 0 for an empty row.
 * s_b has N entries (a per-tensor scale repeated). */
void oracle_row_mean(const int32_t* acc, int64_t ldacc, const float* a_scale,
                     const int32_t* row_ptr, int32_t n_block_rows, int32_t M, int32_t N,
                     const float* s_b, float* out, int64_t ldout) {
  for (int32_t r = 0; r < n_block_rows; ++r) {
    const int32_t rb = row_ptr[r], re = row_ptr[r + 1];
    for (int32_t n = 0; n < N; ++n) {
      float S = 0.0f;
      for (int32_t t = rb; t < re; ++t) {
        const float prod = a_scale[t] * s_b[n];
        S = S + prod;
      }
      const float avg = (re > rb) ? S / (float)(re - rb) : 0.0f;
      for (int i = 0; i < TILE; ++i) {
        const int64_t m = (int64_t)r * TILE + i;
        if (m >= M) break;
        out[m * ldout + n] = (re > rb) ? (float)acc[m * ldacc + n] * avg : 0.0f;
      }
    }
  }
}

/* True per-tile dequantisation in double:
 *   out[m][n] = s_b[n] * sum_t s_a[t] * (A_t @ B)[m][n],  each tile product exact. */
void oracle_i8_per_block(const int8_t* tiles, const float* a_scale, const int32_t* row_ptr,
                         const int32_t* col_idx, int32_t n_block_rows, int32_t M, int32_t K,
                         const int8_t* b, int64_t ldb, int32_t N, const float* s_b,
                         double* out, int64_t ldout) {
#pragma omp parallel for schedule(dynamic, 1)
  for (int32_t r = 0; r < n_block_rows; ++r) {
    int64_t part[TILE][512];
    double sum[TILE][512];
    for (int32_t n0 = 0; n0 < N; n0 += 512) {
      const int32_t nn = (N - n0) < 512 ? (N - n0) : 512;
      for (int i = 0; i < TILE; ++i)
        for (int32_t n = 0; n < nn; ++n) sum[i][n] = 0.0;
      for (int32_t t = row_ptr[r]; t < row_ptr[r + 1]; ++t) {
        const int8_t* tile = tiles + (int64_t)t * TILE * TILE;
        for (int i = 0; i < TILE; ++i) memset(part[i], 0, sizeof(int64_t) * (size_t)nn);
        for (int k = 0; k < TILE; ++k) {
          const int64_t kk = (int64_t)col_idx[t] * TILE + k;
          if (kk >= K) break;
          const int8_t* brow = b + kk * ldb + n0;
          for (int i = 0; i < TILE; ++i) {
            const int64_t av = tile[i * TILE + k];
            if (av == 0) continue;
            for (int32_t n = 0; n < nn; ++n) part[i][n] += av * (int64_t)brow[n];
          }
        }
        const double s = (double)a_scale[t];
        for (int i = 0; i < TILE; ++i)
          for (int32_t n = 0; n < nn; ++n) sum[i][n] += s * (double)part[i][n];
      }
      for (int i = 0; i < TILE; ++i) {
        const int64_t m = (int64_t)r * TILE + i;
        if (m >= M) break;
        for (int32_t n = 0; n < nn; ++n) out[m * ldout + n0 + n] = sum[i][n] * (double)s_b[n0 + n];
      }
    }
  }
}

/* OCP E4M3FN: 1 sign, 4 exponent (bias 7), 3 mantissa bits; no infinities;
 * S.1111.111 is NaN; exponent 0 encodes subnormals m/8 * 2^-6. */
double oracle_e4m3_decode(uint8_t v) {
  const int s = v >> 7, e = (v >> 3) & 15, m = v & 7;
  double x;
  if (e == 15 && m == 7) return NAN;
  if (e == 0) x = ldexp((double)m / 8.0, -6);
  else x = ldexp(1.0 + (double)m / 8.0, e - 7);
  return s ? -x : x;
}

/* E4M3 SpMM in double with a B given as doubles:
 * out[m][n] = s_b[n] * sum_t s_a[t] * sum_k dec(A_t[i][k]) b[kk][n]. */
static void fp8_spmm_dense_b(const uint8_t* tiles, const float* a_scale, const int32_t* row_ptr,
                             const int32_t* col_idx, int32_t n_block_rows, int32_t M, int32_t K,
                             const double* b, int64_t ldb, int32_t N, const float* s_b, double* out,
                             int64_t ldout) {
  double lut[256];
  for (int v = 0; v < 256; ++v) lut[v] = oracle_e4m3_decode((uint8_t)v);
#pragma omp parallel for schedule(dynamic, 1)
  for (int32_t r = 0; r < n_block_rows; ++r) {
    double part[TILE][512];
    double sum[TILE][512];
    for (int32_t n0 = 0; n0 < N; n0 += 512) {
      const int32_t nn = (N - n0) < 512 ? (N - n0) : 512;
      for (int i = 0; i < TILE; ++i)
        for (int32_t n = 0; n < nn; ++n) sum[i][n] = 0.0;
      for (int32_t t = row_ptr[r]; t < row_ptr[r + 1]; ++t) {
        const uint8_t* tile = tiles + (int64_t)t * TILE * TILE;
        for (int i = 0; i < TILE; ++i)
          for (int32_t n = 0; n < nn; ++n) part[i][n] = 0.0;
        for (int k = 0; k < TILE; ++k) {
          const int64_t kk = (int64_t)col_idx[t] * TILE + k;
          if (kk >= K) break;
          const double* brow = b + kk * ldb + n0;
          for (int i = 0; i < TILE; ++i) {
            const double av = lut[tile[i * TILE + k]];
            if (av == 0.0) continue;
            for (int32_t n = 0; n < nn; ++n) part[i][n] += av * brow[n];
          }
        }
        const double s = (double)a_scale[t];
        for (int i = 0; i < TILE; ++i)
          for (int32_t n = 0; n < nn; ++n) sum[i][n] += s * part[i][n];
      }
      for (int i = 0; i < TILE; ++i) {
        const int64_t m = (int64_t)r * TILE + i;
        if (m >= M) break;
        for (int32_t n = 0; n < nn; ++n) out[m * ldout + n0 + n] = sum[i][n] * (double)s_b[n0 + n];
      }
    }
  }
}

/* FP8 SpMM in double: out[m][n] = s_b[n] * sum_t s_a[t] * sum_k dec(A_t[i][k]) dec(B[kk][n])
 * (fp8.py:624-659 with the fp32 upcast replaced by exact doubles).  Returns 0,
 * or -1 when the decoded copy of B cannot be allocated. */
int oracle_fp8_spmm(const uint8_t* tiles, const float* a_scale, const int32_t* row_ptr,
                    const int32_t* col_idx, int32_t n_block_rows, int32_t M, int32_t K,
                    const uint8_t* b, int64_t ldb, int32_t N, const float* s_b, double* out,
                    int64_t ldout) {
  double lut[256];
  for (int v = 0; v < 256; ++v) lut[v] = oracle_e4m3_decode((uint8_t)v);
  double* bd = (double*)malloc(sizeof(double) * ((size_t)K * (size_t)N + 1));
  if (!bd) return -1;
  for (int64_t k = 0; k < K; ++k)
    for (int32_t n = 0; n < N; ++n) bd[k * N + n] = lut[b[k * ldb + n]];
  fp8_spmm_dense_b(tiles, a_scale, row_ptr, col_idx, n_block_rows, M, K, bd, N, N, s_b, out, ldout);
  free(bd);
  return 0;
}

/* The reference's FP8 SpMM with a float B (fp8.py:624-671: A upcast to fp32
 * and scaled per tile, B upcast to fp32, fp32 dot), in double:
 * out[m][n] = s_b[n] * sum_t s_a[t] * sum_k dec(A_t[i][k]) B[kk][n], B fp32. */
int oracle_fp8_spmm_f32b(const uint8_t* tiles, const float* a_scale, const int32_t* row_ptr,
                         const int32_t* col_idx, int32_t n_block_rows, int32_t M, int32_t K,
                         const float* b, int64_t ldb, int32_t N, const float* s_b, double* out,
                         int64_t ldout) {
  double* bd = (double*)malloc(sizeof(double) * ((size_t)K * (size_t)N + 1));
  if (!bd) return -1;
  for (int64_t k = 0; k < K; ++k)
    for (int32_t n = 0; n < N; ++n) bd[k * N + n] = (double)b[k * ldb + n];
  fp8_spmm_dense_b(tiles, a_scale, row_ptr, col_idx, n_block_rows, M, K, bd, N, N, s_b, out, ldout);
  free(bd);
  return 0;
}

/* tanh-form GELU of fusion.py:38-43 in double: 2 sigmoid(2u) - 1 = tanh(u). */
double oracle_gelu_tanh(double x) {
  const double u = 0.7978845608 * (x + 0.044715 * x * x * x);
  return 0.5 * x * (1.0 + tanh(u));
}

void oracle_gelu_tanh_array(const double* x, double* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = oracle_gelu_tanh(x[i]);
}
