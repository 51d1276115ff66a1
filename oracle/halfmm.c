/* Exact float16 matrix product as NumPy computes it without BLAS — test infrastructure.
 *
 * NumPy has no BLAS path for float16: `a @ b` runs its own inner loop, which widens
 * each element to float32, accumulates a[m,k]·b[k,n] in float32 in increasing k, and
 * rounds the sum once to float16 (round to nearest even). This file computes the same
 * thing, so the oracle's float16 GEMMs (every `@` of the reference's fp16 path:
 * neural_network/_fused_arrays.py:69-71,105,200-205, kernels/fused_sdpa.py:71-78,
 * models/gpt.py:150-153) are bit-exact with the reference and fast enough for the
 * benchmark-sized configs. The product of two float16 values is exact in float32
 * (11 + 11 significand bits), so a fused multiply-add gives the same running sum as a
 * multiply and an add.
 *
 * Only the oracle (tests, fixture scripts) loads this; the product path never does.
 */
#include <immintrin.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* Strided float16 matrix (rows × cols, element (r, c) at src[r·sr + c·sc]) → dense
 * row-major float32. */
static void widen(const uint16_t* src, long rows, long cols, long sr, long sc, float* dst) {
  const int par = (double)rows * cols > 1e6;
  if (sc != 1 && sr == 1) {
    /* column-major source (a transposed view): 64 × 64 blocks, read along columns */
    const long rb = (rows + 63) / 64, cb = (cols + 63) / 64;
#pragma omp parallel for collapse(2) schedule(static) if (par)
    for (long bi = 0; bi < rb; ++bi)
      for (long bj = 0; bj < cb; ++bj) {
        const long r1 = bi * 64 + 64 < rows ? bi * 64 + 64 : rows;
        const long c1 = bj * 64 + 64 < cols ? bj * 64 + 64 : cols;
        for (long c = bj * 64; c < c1; ++c)
          for (long r = bi * 64; r < r1; ++r) dst[r * cols + c] = _cvtsh_ss(src[r + c * sc]);
      }
    return;
  }
#pragma omp parallel for schedule(static) if (par)
  for (long r = 0; r < rows; ++r) {
    const uint16_t* s = src + r * sr;
    float* d = dst + r * cols;
    long c = 0;
    if (sc == 1) {
      for (; c + 8 <= cols; c += 8)
        _mm256_storeu_ps(d + c, _mm256_cvtph_ps(_mm_loadu_si128((const __m128i*)(s + c))));
    }
    for (; c < cols; ++c) d[c] = _cvtsh_ss(s[c * sc]);
  }
}

/* One output row band: rows [m0, m0+mr) × columns [n0, n0+16) with 16-wide vectors,
 * k in increasing order. */
#define MR 6
static void tile6x16(const float* A, long K, const float* B, long N, float* C, long m0, long n0) {
  __m256 c[MR][2];
  for (int i = 0; i < MR; ++i) c[i][0] = c[i][1] = _mm256_setzero_ps();
  const float* a = A + m0 * K;
  for (long k = 0; k < K; ++k) {
    const __m256 b0 = _mm256_loadu_ps(B + k * N + n0);
    const __m256 b1 = _mm256_loadu_ps(B + k * N + n0 + 8);
    for (int i = 0; i < MR; ++i) {
      const __m256 av = _mm256_broadcast_ss(a + i * K + k);
      c[i][0] = _mm256_fmadd_ps(av, b0, c[i][0]);
      c[i][1] = _mm256_fmadd_ps(av, b1, c[i][1]);
    }
  }
  for (int i = 0; i < MR; ++i) {
    _mm256_storeu_ps(C + (m0 + i) * N + n0, c[i][0]);
    _mm256_storeu_ps(C + (m0 + i) * N + n0 + 8, c[i][1]);
  }
}

static void edge(const float* A, long K, const float* B, long N, float* C, long m, long n) {
  float acc = 0.0f;
  for (long k = 0; k < K; ++k) acc = __builtin_fmaf(A[m * K + k], B[k * N + n], acc);
  C[m * N + n] = acc;
}

/* C (M×N float16, element (m, n) at c[m·scm + n·scn]) = a (M×K) · b (K×N), both float16
 * with element strides (sam, sak) and (sbk, sbn). Returns 0, or -1 if out of memory. */
int halfmm(const uint16_t* a, long sam, long sak, const uint16_t* b, long sbk, long sbn,
           uint16_t* c, long scm, long scn, long M, long N, long K) {
  float* A = (float*)malloc(sizeof(float) * (size_t)(M * K + 1));
  float* B = (float*)malloc(sizeof(float) * (size_t)(K * N + 1));
  float* C = (float*)malloc(sizeof(float) * (size_t)(M * N + 1));
  if (!A || !B || !C) {
    free(A);
    free(B);
    free(C);
    return -1;
  }
  widen(a, M, K, sam, sak, A);
  widen(b, K, N, sbk, sbn, B);
  const long mt = M / MR, nt = N / 16;
  const int par = (double)M * N * K > 4e6;  /* threads only where they pay */
#pragma omp parallel for collapse(2) schedule(dynamic, 4) if (par)
  for (long i = 0; i < mt; ++i)
    for (long j = 0; j < nt; ++j) tile6x16(A, K, B, N, C, i * MR, j * 16);
#pragma omp parallel for schedule(static) if (par)
  for (long m = 0; m < M; ++m) {
    const long n_start = m < mt * MR ? nt * 16 : 0;
    for (long n = n_start; n < N; ++n) edge(A, K, B, N, C, m, n);
  }
#pragma omp parallel for schedule(static) if (par)
  for (long m = 0; m < M; ++m) {
    uint16_t* out = c + m * scm;
    const float* src = C + m * N;
    long n = 0;
    if (scn == 1) {
      for (; n + 8 <= N; n += 8)
        _mm_storeu_si128((__m128i*)(out + n),
                         _mm256_cvtps_ph(_mm256_loadu_ps(src + n), _MM_FROUND_TO_NEAREST_INT));
    }
    for (; n < N; ++n) out[n * scn] = _cvtss_sh(src[n], _MM_FROUND_TO_NEAREST_INT);
  }
  free(A);
  free(B);
  free(C);
  return 0;
}
