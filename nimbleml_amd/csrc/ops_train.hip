// Backward of compute_loss on the device: the GEMM of the backward's transposed products,
// and the backward of RMSNorm, GELU (fused into a GEMM epilogue), the cross-entropy, causal
// attention, RoPE and the embeddings, plus the column sums behind the bias and gain
// gradients. Every kernel takes the model's storage type T (float or fp16): fp16 operands
// are widened to fp32 on load (products of fp16 values are exact in fp32, as in NumPy's
// fp16 matmul with fp32 accumulation), activation gradients are stored in T, parameter
// gradients accumulate in fp32, and the fp16 branches keep the reference's fp16 rounding
// points where the reference writes them op by op (RMSNorm, GELU, cross-entropy, RoPE).
//
//  * gemm_bwd_kernel: 128 × 128 tile, 4 waves of 64 × 64, MFMA 32×32×2 fp32; either
//    operand read k-contiguous (rows of a row-major matrix) or m/n-contiguous (columns),
//    staged through LDS as [k][row] so every MFMA fragment read is a contiguous row.
//  * attention backward: per (sequence, head), one kernel owns a tile of keys and
//    walks the queries after it (dK, dV), another owns a tile of queries and walks the
//    keys before it (dQ); both recompute P = exp(q·k/√dk − lse) from the forward's
//    log-sum-exp, so no (S × S) matrix is kept.
//  * reductions over rows (bias / gain gradients) go through per-block partial rows
//    and a second pass in a fixed order: the result does not depend on scheduling.
#include <cstdlib>

#include "gemm_big.hpp"
#include "kernels.hpp"

namespace nml {

namespace {

// 4 consecutive elements as fp32 (16-byte float or 8-byte fp16 load) and back.
template <typename T>
__device__ __forceinline__ floatx4 ld4(const T* p) {
  if constexpr (sizeof(T) == 4) {
    return *reinterpret_cast<const floatx4*>(p);
  } else {
    const half4 h = *reinterpret_cast<const half4*>(p);
    const floatx4 v = {static_cast<float>(h[0]), static_cast<float>(h[1]), static_cast<float>(h[2]),
                       static_cast<float>(h[3])};
    return v;
  }
}
template <typename T>
__device__ __forceinline__ void st4(T* p, floatx4 v) {
  if constexpr (sizeof(T) == 4) {
    *reinterpret_cast<floatx4*>(p) = v;
  } else {
    const half4 h = {static_cast<half_t>(v[0]), static_cast<half_t>(v[1]), static_cast<half_t>(v[2]),
                     static_cast<half_t>(v[3])};
    *reinterpret_cast<half4*>(p) = h;
  }
}

// ------------------------------------------------------------------ backward GEMM
constexpr int kGM = 128, kGK = 16, kGPad = 4;
constexpr int kGBPart = 3;  // split-K partial: fp32, unrounded

// gelu'(x) of native/src/gelu.cpp:23-33 (tanh recomputed from x as the forward did).
__device__ __forceinline__ float gelu_grad(float x) {
#pragma clang fp contract(off)
  const float x3 = x * x * x;
  const float tu = tanhf(0.7978845608028654f * (x + 0.044715f * x3));
  const float du_dx = 0.7978845608028654f * (1.0f + 0.134145f * x * x);
  const float sech2 = 1.0f - tu * tu;
  return 0.5f * (1.0f + tu) + 0.5f * x * sech2 * du_dx;
}

// fp16: g·gelu'(x) in the fp16 ops of kernels/fused_gelu.py:97-102 (tu as the fp16 forward
// forms it, kernels/fused_gelu.py:67; each product and sum rounded to fp16).
// The factor gelu'(x) of the fp16 branch, a function of the fp16 x alone;
// gelu_grad_f16(g, x) = fp16(g · factor).
__device__ __forceinline__ float gelu_grad_f16_factor(float x) {
#pragma clang fp contract(off)
  const float k = static_cast<float>(static_cast<half_t>(0.7978845608028654f));
  const float c = static_cast<float>(static_cast<half_t>(0.044715f));
  const float dc = static_cast<float>(static_cast<half_t>(0.134145f));
  float t = rnd<half_t>(c * x);
  t = rnd<half_t>(t * x);
  t = rnd<half_t>(t * x);
  t = rnd<half_t>(x + t);
  t = rnd<half_t>(k * t);
  const float tu = rnd<half_t>(tanh_h(t));
  float du = rnd<half_t>(dc * x);
  du = rnd<half_t>(du * x);
  du = rnd<half_t>(1.0f + du);
  du = rnd<half_t>(k * du);
  const float sech2 = rnd<half_t>(1.0f - rnd<half_t>(tu * tu));
  const float a = rnd<half_t>(0.5f * rnd<half_t>(1.0f + tu));
  float b = rnd<half_t>(0.5f * x);
  b = rnd<half_t>(b * sech2);
  b = rnd<half_t>(b * du);
  return rnd<half_t>(a + b);
}

__device__ __forceinline__ float gelu_grad_f16(float g, float x) {
#pragma clang fp contract(off)
  return rnd<half_t>(g * gelu_grad_f16_factor(x));
}

// gelu_grad_f16_factor of every fp16 x, indexed by its bit pattern (128 KiB, L2-resident):
// the direct-to-LDS backward GEMM's GELU epilogue reads the factor with one load instead
// of ~70 VALU instructions. Filled from gelu_grad_f16_factor itself.
__device__ half_t g_dgelu16_tab[65536];

__global__ __launch_bounds__(256) void dgelu16_tab_kernel() {
  const int i = blockIdx.x * 256 + threadIdx.x;
  const half_t x = __builtin_bit_cast(half_t, static_cast<uint16_t>(i));
  g_dgelu16_tab[i] = static_cast<half_t>(gelu_grad_f16_factor(static_cast<float>(x)));
}

// Once per device before the first use (training is never captured).
int dgelu16_tab_ready(hipStream_t st) {
  static bool done[64] = {};
  int dev = 0;
  NML_HIP(hipGetDevice(&dev));
  if (dev >= 0 && dev < 64 && done[dev]) return 0;
  dgelu16_tab_kernel<<<256, 256, 0, st>>>();
  NML_LAUNCHED();
  NML_HIP(hipStreamSynchronize(st));
  if (dev >= 0 && dev < 64) done[dev] = true;
  return 0;
}

// One operand tile (128 rows × 16 k) into LDS as S[k][row]. KC: element (r, k) at
// p[r·ld + k] (4 lanes per row, 16-byte loads along k, transposed on the LDS store);
// otherwise at p[k·ld + r] (32 lanes per k row, 16-byte loads and stores). Out-of-range
// rows / k read as 0. Two 16-byte vectors per thread.
template <bool KC, typename T>
__device__ __forceinline__ void tile_load(const T* __restrict__ p, long long ld, int r0,
                                          int R, int k0, int K, floatx4 (&v)[2]) {
  const int tid = threadIdx.x;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int c = tid + 256 * i;
    const floatx4 zero = {0.f, 0.f, 0.f, 0.f};
    if constexpr (KC) {
      const int row = c >> 2, kc = (c & 3) * 4;
      const bool ok = r0 + row < R && k0 + kc < K;
      v[i] = ok ? ld4(p + static_cast<long long>(r0 + row) * ld + k0 + kc) : zero;
    } else {
      const int kr = c >> 5, rc = (c & 31) * 4;
      const bool ok = k0 + kr < K && r0 + rc < R;
      v[i] = ok ? ld4(p + static_cast<long long>(k0 + kr) * ld + r0 + rc) : zero;
    }
  }
}

template <bool KC>
__device__ __forceinline__ void tile_store(float (*S)[kGM + kGPad], const floatx4 (&v)[2]) {
  const int tid = threadIdx.x;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int c = tid + 256 * i;
    if constexpr (KC) {
      const int row = c >> 2, kc = (c & 3) * 4;
#pragma unroll
      for (int j = 0; j < 4; ++j) S[kc + j][row] = v[i][j];
    } else {
      const int kr = c >> 5, rc = (c & 31) * 4;
      *reinterpret_cast<floatx4*>(&S[kr][rc]) = v[i];
    }
  }
}

// Split K (gridDim.z > 1): block z multiplies k in [z·kchunk, (z + 1)·kchunk) and writes
// its partial product to c + z·zstride (OUT = GB_SET), summed afterwards in a fixed order.
// T: operand type (and the output type of GB_SET / GB_GELU); GB_ADD adds fp32(T(acc)) to
// an fp32 output (the reference forms the gradient in T, then accumulates it in fp32).
template <bool A_KC, bool B_KC, int OUT, typename T>
__global__ __launch_bounds__(256) void gemm_bwd_kernel(GemmBwdArgs g, int kchunk, long long zstride) {
  __shared__ __attribute__((aligned(16))) float As[kGK][kGM + kGPad];
  __shared__ __attribute__((aligned(16))) float Bs[kGK][kGM + kGPad];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int m0 = blockIdx.y * kGM, n0 = blockIdx.x * kGM;
  const int M = g.M, N = g.N;
  const int kbeg = blockIdx.z * kchunk;
  const int K = min(g.K, kbeg + kchunk);
  const T* __restrict__ ga = static_cast<const T*>(g.a);
  const T* __restrict__ gbp = static_cast<const T*>(g.b);

  floatx16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  floatx4 ra[2], rb[2];
  tile_load<A_KC>(ga, g.lda, m0, M, kbeg, K, ra);
  tile_load<B_KC>(gbp, g.ldb, n0, N, kbeg, K, rb);
  tile_store<A_KC>(As, ra);
  tile_store<B_KC>(Bs, rb);
  __syncthreads();
  for (int k0 = kbeg; k0 < K; k0 += kGK) {
    const bool more = k0 + kGK < K;
    if (more) {  // next tile's loads in flight while this one multiplies
      tile_load<A_KC>(ga, g.lda, m0, M, k0 + kGK, K, ra);
      tile_load<B_KC>(gbp, g.ldb, n0, N, k0 + kGK, K, rb);
    }
#pragma unroll
    for (int kk = 0; kk < kGK; kk += 2) {
      float fa[2], fb[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) fa[i] = As[kk + (lane >> 5)][wm * 64 + i * 32 + (lane & 31)];
#pragma unroll
      for (int j = 0; j < 2; ++j) fb[j] = Bs[kk + (lane >> 5)][wn * 64 + j * 32 + (lane & 31)];
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[i], fb[j], acc[i][j], 0, 0, 0);
    }
    __syncthreads();
    if (more) {
      tile_store<A_KC>(As, ra);
      tile_store<B_KC>(Bs, rb);
    }
    __syncthreads();
  }

  // D layout of a 32×32 MFMA tile: lane l, register r → row 8(r/4) + 4(l/32) + r%4, col l%32.
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = m0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        const int n = n0 + wn * 64 + j * 32 + (lane & 31);
        if (m < M && n < N) {
          const long long ci = blockIdx.z * zstride + static_cast<long long>(m) * g.ldc + n;
          const float v = acc[i][j][r];
          if constexpr (OUT == kGBPart) {
            static_cast<float*>(g.c)[ci] = v;
          } else if constexpr (OUT == GB_ADD) {
            static_cast<float*>(g.c)[ci] += rnd<T>(v);
          } else if constexpr (OUT == GB_SET) {
            static_cast<T*>(g.c)[ci] = static_cast<T>(v);
          } else {
            const float x = static_cast<float>(static_cast<const T*>(g.aux)[static_cast<long long>(m) * g.ldaux + n]);
            if constexpr (sizeof(T) == 4)
              static_cast<T*>(g.c)[ci] = v * gelu_grad(x);
            else
              static_cast<T*>(g.c)[ci] = static_cast<T>(gelu_grad_f16(rnd<T>(v), x));
          }
        }
      }
}

// ---- fp16 operands on the fp16 MFMA (32×32×16, fp32 accumulation): 128 × 128 tiles,
// 32-wide k tiles, 4 waves of 64 × 64. LDS holds each operand as [row][k] (k contiguous, a
// 16-byte fragment per lane and k step); k-contiguous operands are copied in 16-byte
// pieces, the others (8 consecutive rows at one k per piece) are transposed on the store.
constexpr int kHK16 = 64, kHP16 = kHK16 + 8;  // k tile, LDS row pitch (halves)
constexpr int kHV16 = kGM * kHK16 / 8 / 256;    // 16-byte pieces per thread per operand tile

template <bool KC>
__device__ __forceinline__ void tile16_load(const half_t* __restrict__ p, long long ld, int r0,
                                            int R, int k0, int K, half8 (&v)[kHV16]) {
  const half8 z = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
  for (int i = 0; i < kHV16; ++i) {
    const int c = threadIdx.x + 256 * i;
    if constexpr (KC) {
      const int row = c / (kHK16 / 8), kc = (c % (kHK16 / 8)) * 8;
      const bool ok = r0 + row < R && k0 + kc < K;
      v[i] = ok ? *reinterpret_cast<const half8*>(p + static_cast<long long>(r0 + row) * ld + k0 + kc) : z;
    } else {
      // a 4 (k) × 8 (rows) block per thread: rows 8·(t % 16)…, k 4·(t / 16) + i
      const int rb = (threadIdx.x & 15) * 8, kr = (threadIdx.x >> 4) * 4 + i;
      const bool ok = k0 + kr < K && r0 + rb < R;
      v[i] = ok ? *reinterpret_cast<const half8*>(p + static_cast<long long>(k0 + kr) * ld + r0 + rb) : z;
    }
  }
}

template <bool KC>
__device__ __forceinline__ void tile16_store(half_t (*S)[kHP16], const half8 (&v)[kHV16]) {
#pragma unroll
  for (int i = 0; i < kHV16; ++i) {
    const int c = threadIdx.x + 256 * i;
    if constexpr (KC) {
      const int row = c / (kHK16 / 8), kc = (c % (kHK16 / 8)) * 8;
      *reinterpret_cast<half8*>(&S[row][kc]) = v[i];
    } else if (i == 0) {  // the 4 × 8 block transposed in registers: one 8-byte store per row
      const int rb = (threadIdx.x & 15) * 8, kq = (threadIdx.x >> 4) * 4;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const half4 w = {v[0][j], v[1][j], v[2][j], v[3][j]};
        *reinterpret_cast<half4*>(&S[rb + j][kq]) = w;
      }
    }
  }
}

template <bool A_KC, bool B_KC, int OUT>
__global__ __launch_bounds__(256) void gemm_bwd_f16_kernel(GemmBwdArgs g, int kchunk, long long zstride) {
  __shared__ __attribute__((aligned(16))) half_t As[kGM][kHP16];
  __shared__ __attribute__((aligned(16))) half_t Bs[kGM][kHP16];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int m0 = blockIdx.y * kGM, n0 = blockIdx.x * kGM;
  const int M = g.M, N = g.N;
  const int kbeg = blockIdx.z * kchunk;
  const int K = min(g.K, kbeg + kchunk);
  const half_t* __restrict__ ga = static_cast<const half_t*>(g.a);
  const half_t* __restrict__ gbp = static_cast<const half_t*>(g.b);

  floatx16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  half8 ra[kHV16], rb[kHV16];
  tile16_load<A_KC>(ga, g.lda, m0, M, kbeg, K, ra);
  tile16_load<B_KC>(gbp, g.ldb, n0, N, kbeg, K, rb);
  tile16_store<A_KC>(As, ra);
  tile16_store<B_KC>(Bs, rb);
  __syncthreads();
  const int fr = lane & 31, fk = (lane >> 5) * 8;
  for (int k0 = kbeg; k0 < K; k0 += kHK16) {
    const bool more = k0 + kHK16 < K;
    if (more) {  // next tile's loads in flight while this one multiplies
      tile16_load<A_KC>(ga, g.lda, m0, M, k0 + kHK16, K, ra);
      tile16_load<B_KC>(gbp, g.ldb, n0, N, k0 + kHK16, K, rb);
    }
#pragma unroll
    for (int ks = 0; ks < kHK16; ks += 16) {
      half8 fa[2], fb[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) fa[i] = *reinterpret_cast<const half8*>(&As[wm * 64 + i * 32 + fr][ks + fk]);
#pragma unroll
      for (int j = 0; j < 2; ++j) fb[j] = *reinterpret_cast<const half8*>(&Bs[wn * 64 + j * 32 + fr][ks + fk]);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa[i], fb[j], acc[i][j], 0, 0, 0);
    }
    __syncthreads();
    if (more) {
      tile16_store<A_KC>(As, ra);
      tile16_store<B_KC>(Bs, rb);
    }
    __syncthreads();
  }

#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = m0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        const int n = n0 + wn * 64 + j * 32 + (lane & 31);
        if (m < M && n < N) {
          const long long ci = blockIdx.z * zstride + static_cast<long long>(m) * g.ldc + n;
          const float v = acc[i][j][r];
          if constexpr (OUT == kGBPart) {
            static_cast<float*>(g.c)[ci] = v;
          } else if constexpr (OUT == GB_ADD) {
            static_cast<float*>(g.c)[ci] += rnd<half_t>(v);
          } else if constexpr (OUT == GB_SET) {
            static_cast<half_t*>(g.c)[ci] = static_cast<half_t>(v);
          } else {
            const float x = static_cast<float>(static_cast<const half_t*>(g.aux)[static_cast<long long>(m) * g.ldaux + n]);
            static_cast<half_t*>(g.c)[ci] = static_cast<half_t>(gelu_grad_f16(rnd<half_t>(v), x));
          }
        }
      }
}

// c[m·ldc + n] += T(Σ_z part[z·M·N + m·N + n]), z in order.
template <typename T>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float* __restrict__ part, int splits,
                                                            int M, int N, float* __restrict__ c,
                                                            long long ldc) {
  const long long i = static_cast<long long>(blockIdx.x) * 256 + threadIdx.x;
  const long long mn = static_cast<long long>(M) * N;
  if (i >= mn) return;
  float s = 0.f;
  for (int z = 0; z < splits; ++z) s += part[z * mn + i];
  const int m = static_cast<int>(i / N), n = static_cast<int>(i - static_cast<long long>(m) * N);
  c[static_cast<long long>(m) * ldc + n] += rnd<T>(s);
}

// Split-K partials of the weight-gradient GEMMs (grow-only; training is never captured).
struct SplitWs {
  float* p = nullptr;
  size_t floats = 0;
};
SplitWs g_split;

// ------------------------------------------- float16 backward GEMM on big::mainloop
// The backward's products read one operand (dX = dY·W: W) or both (dW = dYᵀ·X) across k.
// Those operands are first transposed into a workspace (transpose16_kernel, HBM-bound,
// a few µs per weight) so that both are k-contiguous rows, and the product then runs on
// the prefill GEMM's direct-to-LDS main loop: 256 × 256 tiles where they fill the chip,
// 128 × 128 tiles (two workgroups per CU) otherwise, and split K for the weight
// gradients whose output tiles are few.

// dst[c·ldd + r] = src[r·lds + c] for r < rows, c < cols (fp16; rows and cols multiples
// of 8, strides multiples of 8, both 16-byte aligned); one 64 × 64 tile per workgroup.
// Up to two such transposes in one launch (grid z = the job; a workgroup past its job's
// extent returns), so a product that reads both operands across k pays one launch.
struct Transpose16Job {
  const half_t* src;
  long long lds;
  int rows, cols;
  half_t* dst;
  long long ldd;
};

__global__ __launch_bounds__(256) void transpose16_kernel(Transpose16Job j0, Transpose16Job j1) {
  __shared__ half_t t[64][66];  // row stride 132 bytes: column reads spread over the banks
  const Transpose16Job& j = blockIdx.z == 0 ? j0 : j1;
  const half_t* __restrict__ src = j.src;
  half_t* __restrict__ dst = j.dst;
  const long long lds = j.lds, ldd = j.ldd;
  const int rows = j.rows, cols = j.cols;
  const int r0 = blockIdx.y * 64, c0 = blockIdx.x * 64, tid = threadIdx.x;
  if (r0 >= rows || c0 >= cols) return;  // (uniform over the workgroup)
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int p = tid + 256 * i, r = p >> 3, c8 = (p & 7) * 8;
    if (r0 + r < rows && c0 + c8 < cols) {
      const half8 v = *reinterpret_cast<const half8*>(src + static_cast<long long>(r0 + r) * lds + c0 + c8);
#pragma unroll
      for (int e = 0; e < 8; ++e) t[r][c8 + e] = v[e];
    }
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int p = tid + 256 * i, c = p >> 3, r8 = (p & 7) * 8;
    if (c0 + c < cols && r0 + r8 < rows) {
      half8 v;
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = t[r8 + e][c];
      *reinterpret_cast<half8*>(dst + static_cast<long long>(c0 + c) * ldd + r0 + r8) = v;
    }
  }
}

// c (m, n) = out(Σ_k a[m·lda + k] · b[n·ldb + k]) over this split's k range, output modes
// as gemm_bwd_f16_kernel. Workgroup b → (split, tile) through the XCD-aware order;
// `tiles_m` m-tiles per column of tiles.
constexpr int kBwdGM = 8;

template <int TM, int TN, int OUT>
__global__ __launch_bounds__(big::kThreads, TM == 256 ? 1 : 4) void gemm_bwd_big_kernel(
    GemmBwdArgs g, int tiles_m, int tiles, int splits, int kchunk, long long zstride) {
  extern __shared__ __attribute__((aligned(1024))) char lds_raw[];
  constexpr int IA = TM / 64, JB = TN / 128;
  const int u = big::xcd_tile(blockIdx.x, tiles * splits);
  const int z = u % splits, tile = u / splits;
  // Tiles in groups of kBwdGM m-tiles (m fastest inside a group, then n), so that an
  // XCD's contiguous range of tiles is a block of up to kBwdGM rows of tiles by a few
  // columns rather than whole columns: with whole columns (4096 × 1024 outputs: one
  // column of 32 tiles per XCD) every XCD streamed all of A through its L2.
  const int tiles_n = tiles / tiles_m;
  const int group = tile / (kBwdGM * tiles_n), first_m = group * kBwdGM;
  const int gm = min(tiles_m - first_m, kBwdGM);
  const int in_group = tile - group * kBwdGM * tiles_n;
  const int m0 = (first_m + in_group % gm) * TM, n0 = (in_group / gm) * TN;
  const int kbeg = z * kchunk;
  const int klen = min(kchunk, g.K - kbeg);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave >> 2, wn = wave & 3;
  floatx16 acc[IA][JB];
#pragma unroll
  for (int i = 0; i < IA; ++i)
#pragma unroll
    for (int j = 0; j < JB; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
  big::mainloop<TM, TN>(static_cast<const half_t*>(g.a), g.lda, static_cast<const half_t*>(g.b), g.ldb, g.M,
                        g.N, kbeg, klen / big::kK, m0, n0, lds_raw, acc);
  // Epilogue: every load of a 32 × 32 tile (the GELU factors, the accumulated outputs) is
  // issued before the first store, at clamped addresses, so the tile waits once.
#pragma unroll
  for (int i = 0; i < IA; ++i)
#pragma unroll
    for (int j = 0; j < JB; ++j) {
      const int n = n0 + wn * (TN / 4) + j * 32 + (lane & 31);
      const int nc = min(n, g.N - 1);
      const int mb = m0 + wm * (TM / 2) + i * 32 + 4 * (lane >> 5);
      float in[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        in[r] = 0.f;
        if constexpr (OUT == GB_GELU) {
          const int mc = min(mb + 8 * (r >> 2) + (r & 3), g.M - 1);
          const half_t x = static_cast<const half_t*>(g.aux)[static_cast<long long>(mc) * g.ldaux + nc];
          in[r] = static_cast<float>(g_dgelu16_tab[__builtin_bit_cast(uint16_t, x)]);
        } else if constexpr (OUT == GB_ADD) {
          const int mc = min(mb + 8 * (r >> 2) + (r & 3), g.M - 1);
          in[r] = static_cast<const float*>(g.c)[static_cast<long long>(mc) * g.ldc + nc];
        }
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = mb + 8 * (r >> 2) + (r & 3);
        if (m < g.M && n < g.N) {
          const long long ci = z * zstride + static_cast<long long>(m) * g.ldc + n;
          const float v = acc[i][j][r];
          if constexpr (OUT == kGBPart) {
            static_cast<float*>(g.c)[ci] = v;
          } else if constexpr (OUT == GB_ADD) {
            static_cast<float*>(g.c)[ci] = in[r] + rnd<half_t>(v);
          } else if constexpr (OUT == GB_SET) {
            static_cast<half_t*>(g.c)[ci] = static_cast<half_t>(v);
          } else {  // gelu_grad_f16(fp16(v), pre) = fp16(fp16(v) · factor(pre))
            static_cast<half_t*>(g.c)[ci] = static_cast<half_t>(rnd<half_t>(rnd<half_t>(v) * in[r]));
          }
        }
      }
    }
}

// Grow-only device workspaces (training is never captured into a graph).
struct Ws {
  void* p = nullptr;
  size_t bytes = 0;
};
Ws g_tws;  // transposed operands

int ws_ensure(Ws& w, size_t bytes, hipStream_t st) {
  if (bytes <= w.bytes) return 0;
  NML_HIP(hipStreamSynchronize(st));
  if (w.p) NML_HIP(hipFree(w.p));
  w = Ws{};
  NML_HIP(hipMalloc(&w.p, bytes));
  w.bytes = bytes;
  return 0;
}

template <int TM, int TN, int OUT>
int big_bwd_launch(const GemmBwdArgs& g, int splits, int kchunk, long long zstride, hipStream_t st) {
  static bool attr = false;
  const void* fn = reinterpret_cast<const void*>(&gemm_bwd_big_kernel<TM, TN, OUT>);
  if (!attr) {
    NML_HIP(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize,
                                static_cast<int>(big::Shape<TM, TN>::Lds)));
    attr = true;
  }
  const int tiles_m = (g.M + TM - 1) / TM, tiles = tiles_m * ((g.N + TN - 1) / TN);
  gemm_bwd_big_kernel<TM, TN, OUT><<<tiles * splits, big::kThreads, big::Shape<TM, TN>::Lds, st>>>(
      g, tiles_m, tiles, splits, kchunk, zstride);
  NML_LAUNCHED();
  return 0;
}

template <int TM, int TN>
int big_bwd_out(const GemmBwdArgs& g, int out, int splits, int kchunk, long long zstride, hipStream_t st) {
  switch (out) {
    case GB_SET: return big_bwd_launch<TM, TN, GB_SET>(g, splits, kchunk, zstride, st);
    case GB_ADD: return big_bwd_launch<TM, TN, GB_ADD>(g, splits, kchunk, zstride, st);
    case GB_GELU: return big_bwd_launch<TM, TN, GB_GELU>(g, splits, kchunk, zstride, st);
    case kGBPart: return big_bwd_launch<TM, TN, kGBPart>(g, splits, kchunk, zstride, st);
    default: set_error("gemm_bwd: unknown output mode %d", out); return -1;
  }
}

// The float16 product on big::mainloop; K a multiple of big::kK, operands as
// launch_gemm_bwd's 16-byte conditions.
int gemm_bwd_big(const GemmBwdArgs& g0, bool a_kc, bool b_kc, int out, hipStream_t st) {
  if (out == GB_GELU) NML_TRY(dgelu16_tab_ready(st));
  GemmBwdArgs g = g0;
  const long long M = g.M, N = g.N, K = g.K;
  const size_t at = a_kc ? 0 : static_cast<size_t>(M * K), bt = b_kc ? 0 : static_cast<size_t>(N * K);
  if (at + bt) {
    if (ws_ensure(g_tws, (at + bt) * sizeof(half_t), st) != 0) return -1;
    half_t* ws = static_cast<half_t*>(g_tws.p);
    Transpose16Job job[2];
    int jobs = 0, cols = 0;
    if (!a_kc) {  // a: (k, m) at a[k·lda + m]
      job[jobs++] = Transpose16Job{static_cast<const half_t*>(g.a), g.lda, static_cast<int>(K),
                                   static_cast<int>(M), ws, K};
      cols = static_cast<int>(M);
      g.a = ws;
      g.lda = K;
    }
    if (!b_kc) {  // b: (k, n) at b[k·ldb + n]
      job[jobs++] = Transpose16Job{static_cast<const half_t*>(g.b), g.ldb, static_cast<int>(K),
                                   static_cast<int>(N), ws + at, K};
      cols = cols > static_cast<int>(N) ? cols : static_cast<int>(N);
      g.b = ws + at;
      g.ldb = K;
    }
    transpose16_kernel<<<dim3((cols + 63) / 64, static_cast<unsigned>((K + 63) / 64), jobs), 256, 0, st>>>(
        job[0], jobs > 1 ? job[1] : job[0]);
    NML_LAUNCHED();
  }
  // 128 × 128 tiles, two workgroups per CU (256 × 256 tiles measured slower here: the
  // backward's products have at most 4096 × 4096 outputs, one round of large tiles, and
  // the GELU-backward epilogue then overlaps nothing)
  const long long tiles = ((M + 127) / 128) * ((N + 127) / 128);
  // Split K (accumulating outputs only): while the grid is short of one workgroup per CU
  // and each slice keeps ≥ 1024 of k (filling two per CU instead, with the 4096 × 1024
  // weight gradients split in two, measured 1.2 ms slower per C3-sized training step:
  // the partial sums' extra pass costs more than the second workgroup gains).
  int splits = 1;
  if (out == GB_ADD)
    while (splits < 16 && tiles * splits < 256 && K / (2 * splits) >= 1024) splits *= 2;
  const int steps = static_cast<int>(K / big::kK);
  const int kchunk = (steps + splits - 1) / splits * big::kK;
  splits = static_cast<int>((K + kchunk - 1) / kchunk);  // no empty slice
  if (splits == 1) return big_bwd_out<128, 128>(g, out, 1, kchunk, 0, st);
  const size_t need = static_cast<size_t>(splits) * M * N;
  if (need > g_split.floats) {
    NML_HIP(hipStreamSynchronize(st));
    if (g_split.p) NML_HIP(hipFree(g_split.p));
    g_split = SplitWs{};
    NML_HIP(hipMalloc(&g_split.p, need * sizeof(float)));
    g_split.floats = need;
  }
  GemmBwdArgs p = g;
  p.c = g_split.p;
  p.ldc = g.N;
  NML_TRY((big_bwd_out<128, 128>(p, kGBPart, splits, kchunk, M * N, st)));
  splitk_reduce_kernel<half_t><<<static_cast<int>((M * N + 255) / 256), 256, 0, st>>>(
      g_split.p, splits, g.M, g.N, static_cast<float*>(g.c), g.ldc);
  NML_LAUNCHED();
  return 0;
}

template <bool A_KC, bool B_KC, typename T>
int gemm_bwd_out(const GemmBwdArgs& g, int out, hipStream_t st, bool mfma16 = false) {
  const int tn = (g.N + kGM - 1) / kGM, tm = (g.M + kGM - 1) / kGM;
  // Few output tiles and a long K (a weight gradient, K = rows): split K so that the
  // grid holds ≥ 1024 blocks, each K slice ≥ 512 long.
  int splits = 1;
  if (out == GB_ADD) {
    while (splits < 16 && tn * tm * splits < 1024 && g.K / (2 * splits) >= 512) splits *= 2;
  }
  if (splits > 1) {
    const size_t need = static_cast<size_t>(splits) * g.M * g.N;
    if (need > g_split.floats) {
      NML_HIP(hipStreamSynchronize(st));
      if (g_split.p) NML_HIP(hipFree(g_split.p));
      g_split = SplitWs{};
      NML_HIP(hipMalloc(&g_split.p, need * sizeof(float)));
      g_split.floats = need;
    }
    const int kchunk = ((g.K + splits - 1) / splits + kHK16 - 1) / kHK16 * kHK16;
    GemmBwdArgs p = g;
    p.c = g_split.p;
    p.ldc = g.N;
    const dim3 grid(tn, tm, splits);
    if constexpr (sizeof(T) == 2) {
      if (mfma16)
        gemm_bwd_f16_kernel<A_KC, B_KC, kGBPart><<<grid, 256, 0, st>>>(p, kchunk, static_cast<long long>(g.M) * g.N);
      else
        gemm_bwd_kernel<A_KC, B_KC, kGBPart, T><<<grid, 256, 0, st>>>(p, kchunk, static_cast<long long>(g.M) * g.N);
    } else {
      gemm_bwd_kernel<A_KC, B_KC, kGBPart, T><<<grid, 256, 0, st>>>(p, kchunk, static_cast<long long>(g.M) * g.N);
    }
    NML_LAUNCHED();
    const long long mn = static_cast<long long>(g.M) * g.N;
    splitk_reduce_kernel<T><<<static_cast<int>((mn + 255) / 256), 256, 0, st>>>(
        g_split.p, splits, g.M, g.N, static_cast<float*>(g.c), g.ldc);
    NML_LAUNCHED();
    return 0;
  }
  const dim3 grid(tn, tm);
  if constexpr (sizeof(T) == 2) {
    if (mfma16) {
      switch (out) {
        case GB_SET: gemm_bwd_f16_kernel<A_KC, B_KC, GB_SET><<<grid, 256, 0, st>>>(g, g.K, 0); break;
        case GB_ADD: gemm_bwd_f16_kernel<A_KC, B_KC, GB_ADD><<<grid, 256, 0, st>>>(g, g.K, 0); break;
        case GB_GELU: gemm_bwd_f16_kernel<A_KC, B_KC, GB_GELU><<<grid, 256, 0, st>>>(g, g.K, 0); break;
        default: set_error("gemm_bwd: unknown output mode %d", out); return -1;
      }
      NML_LAUNCHED();
      return 0;
    }
  }
  switch (out) {
    case GB_SET: gemm_bwd_kernel<A_KC, B_KC, GB_SET, T><<<grid, 256, 0, st>>>(g, g.K, 0); break;
    case GB_ADD: gemm_bwd_kernel<A_KC, B_KC, GB_ADD, T><<<grid, 256, 0, st>>>(g, g.K, 0); break;
    case GB_GELU: gemm_bwd_kernel<A_KC, B_KC, GB_GELU, T><<<grid, 256, 0, st>>>(g, g.K, 0); break;
    default: set_error("gemm_bwd: unknown output mode %d", out); return -1;
  }
  NML_LAUNCHED();
  return 0;
}

// ------------------------------------------------------------- RMSNorm backward
constexpr int kNormRowsPerBlock = 16;
constexpr int kNormRowsPerWave = 4;  // wave kernel: enough waves to fill the chip at 4k rows

// One block per 16 rows, each thread NC columns c = tid + 256·j. Per row (fp32, the
// order of kernels/fused_rmsnorm.py:208-217): ms = Σx²/d, rms = √(ms + ε),
// gxh = dy·γ, dot = Σ gxh·x, coef = (2/d)·(−½·dot·(ms + ε)^(−3/2)),
// dx = gxh/rms + x·coef; the block's Σ dy·(x/rms) per column goes to part[block].
template <int NC>
__global__ __launch_bounds__(256) void rmsnorm_bwd_kernel(const float* __restrict__ dy,
                                                          const float* __restrict__ x,
                                                          const float* __restrict__ gam,
                                                          float* __restrict__ dx, int acc,
                                                          float* __restrict__ part, int rows,
                                                          int d, float eps) {
#pragma clang fp contract(off)
  __shared__ float red[2][4];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  float gv[NC], gacc[NC];
#pragma unroll
  for (int j = 0; j < NC; ++j) {
    const int c = tid + 256 * j;
    gv[j] = c < d ? gam[c] : 0.f;
    gacc[j] = 0.f;
  }
  const int r0 = blockIdx.x * kNormRowsPerBlock;
  const int r1 = min(rows, r0 + kNormRowsPerBlock);
  for (int r = r0; r < r1; ++r) {
    const float* xr = x + static_cast<long long>(r) * d;
    const float* gr = dy + static_cast<long long>(r) * d;
    float xv[NC], dv[NC], ssq = 0.f, dot = 0.f;
#pragma unroll
    for (int j = 0; j < NC; ++j) {
      const int c = tid + 256 * j;
      xv[j] = c < d ? xr[c] : 0.f;
      dv[j] = c < d ? gr[c] : 0.f;
      ssq += xv[j] * xv[j];
      dot += (dv[j] * gv[j]) * xv[j];
    }
    ssq = wave_sum(ssq);
    dot = wave_sum(dot);
    if (lane == 0) {
      red[0][w] = ssq;
      red[1][w] = dot;
    }
    __syncthreads();
    const float ms = ((red[0][0] + red[0][1]) + (red[0][2] + red[0][3])) / static_cast<float>(d);
    const float rdot = (red[1][0] + red[1][1]) + (red[1][2] + red[1][3]);
    __syncthreads();  // red is rewritten by the next row
    const float rms = sqrtf(ms + eps);
    const float grad_ms = rdot * -0.5f / ((ms + eps) * rms);
    const float coef = (2.0f / static_cast<float>(d)) * grad_ms;
    float* o = dx + static_cast<long long>(r) * d;
#pragma unroll
    for (int j = 0; j < NC; ++j) {
      const int c = tid + 256 * j;
      if (c < d) {
        const float v = (dv[j] * gv[j]) / rms + xv[j] * coef;
        o[c] = acc ? o[c] + v : v;
        gacc[j] += dv[j] * (xv[j] / rms);
      }
    }
  }
#pragma unroll
  for (int j = 0; j < NC; ++j) {
    const int c = tid + 256 * j;
    if (c < d) part[static_cast<long long>(blockIdx.x) * d + c] = gacc[j];
  }
}

// The same with one wave per 4 rows (4 waves per workgroup): a lane keeps NV vectors of
// 4 elements of the row and the row sums are DPP wave sums; the four waves' dγ
// contributions are summed in order through LDS into part[workgroup]. fp16 (kernels/fused_rmsnorm.py:
// 195-206): ms recomputed as the forward forms it (fp16 squares, fp32 sum), inv = fp16(1/rms),
// x̂ = x·inv, dγ += Σ dy·x̂ (fp16 products, fp32 sum), gxh = dy·γ, dot = Σ gxh·x (fp16
// products, fp32 sum), coef = fp16((2/d)·dot·(−½)·(ms + ε)^(−3/2)), dx = gxh·inv + x·coef,
// every product and sum rounded to fp16 (and the residual add too, as grad_mid += …).
template <typename T, int NV>
__global__ __launch_bounds__(256) void rmsnorm_bwd_wave_kernel(const T* __restrict__ dy,
                                                               const T* __restrict__ x,
                                                               const T* __restrict__ gam,
                                                               T* __restrict__ dx, int acc,
                                                               float* __restrict__ part, int rows,
                                                               int d, float eps) {
#pragma clang fp contract(off)
  constexpr bool H = sizeof(T) == 2;
  __shared__ floatx4 red[4][NV * 64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int wv = blockIdx.x * 4 + w;
  const int r0 = wv * kNormRowsPerWave;
  const int nvec = d / 4, r1 = min(rows, r0 + kNormRowsPerWave);  // r1 ≤ r0 past the end
  floatx4 gv[NV], ga[NV];
  const floatx4 z = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int c = lane + 64 * i;
    gv[i] = c < nvec ? ld4(gam + 4 * c) : z;
    ga[i] = z;
  }
  // A row's operands (x, dy and the dx it adds to when accumulating) are loaded in one
  // batch, and the next row's before this one is computed. Every load is unconditional —
  // the column index clamped, columns past the row and dx when not accumulating zeroed by
  // selects — since a load behind a branch is waited for where the branches join.
  floatx4 xv[NV], dv[NV], av[NV], xn[NV], dn[NV], an[NV];
  auto load_row = [&](int r, floatx4 (&xo)[NV], floatx4 (&go)[NV], floatx4 (&ao)[NV]) {
    const T* xr = x + static_cast<long long>(r) * d;
    const T* gr = dy + static_cast<long long>(r) * d;
    const T* orow = dx + static_cast<long long>(r) * d;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int c = lane + 64 * i, cc = c < nvec ? c : nvec - 1;
      xo[i] = ld4(xr + 4 * cc);
      go[i] = ld4(gr + 4 * cc);
      ao[i] = ld4(orow + 4 * cc);  // dx is the output buffer: always readable
    }
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const bool in = lane + 64 * i < nvec;
      xo[i] = in ? xo[i] : z;
      go[i] = in ? go[i] : z;
      ao[i] = (in && acc) ? ao[i] : z;
    }
  };
  if (r0 < r1) load_row(r0, xv, dv, av);
  for (int r = r0; r < r1; ++r) {
    if (r + 1 < r1) load_row(r + 1, xn, dn, an);
    float ssq = 0.f, dot = 0.f;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if constexpr (H) {
          ssq += rnd<T>(xv[i][e] * xv[i][e]);
          dot += rnd<T>(rnd<T>(dv[i][e] * gv[i][e]) * xv[i][e]);
        } else {
          ssq += xv[i][e] * xv[i][e];
          dot += (dv[i][e] * gv[i][e]) * xv[i][e];
        }
      }
    }
    const float ms = wave_sum_dpp(ssq) / static_cast<float>(d);
    const float rdot = wave_sum_dpp(dot);
    const float rms = sqrtf(ms + eps);
    float inv = 0.f, coef;
    if constexpr (H) {
      inv = rnd<T>(1.0f / rms);
      coef = rnd<T>((2.0f / static_cast<float>(d)) * (rdot * -0.5f * powf(ms + eps, -1.5f)));
    } else {
      coef = (2.0f / static_cast<float>(d)) * (rdot * -0.5f / ((ms + eps) * rms));
    }
    T* o = dx + static_cast<long long>(r) * d;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int c = lane + 64 * i;
      floatx4 v = av[i];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if constexpr (H) {
          const float gx = rnd<T>(rnd<T>(rnd<T>(dv[i][e] * gv[i][e]) * inv) + rnd<T>(xv[i][e] * coef));
          v[e] = acc ? rnd<T>(v[e] + gx) : gx;
          ga[i][e] += rnd<T>(dv[i][e] * rnd<T>(xv[i][e] * inv));
        } else {
          v[e] += (dv[i][e] * gv[i][e]) / rms + xv[i][e] * coef;
          ga[i][e] += dv[i][e] * (xv[i][e] / rms);
        }
      }
      if (c < nvec) st4(o + 4 * c, v);
    }
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      xv[i] = xn[i];
      dv[i] = dn[i];
      av[i] = an[i];
    }
  }
#pragma unroll
  for (int i = 0; i < NV; ++i) red[w][lane + 64 * i] = ga[i];
  __syncthreads();
  for (int c = threadIdx.x; c < nvec; c += 256) {
    floatx4 t = red[0][c];
#pragma unroll
    for (int j = 1; j < 4; ++j) {
#pragma unroll
      for (int e = 0; e < 4; ++e) t[e] += red[j][c][e];
    }
    reinterpret_cast<floatx4*>(part + static_cast<long long>(blockIdx.x) * d)[c] = t;
  }
}

// out[c] += Σ_p part[p·n + c]: 32 columns per block, 8 thread rows each summing every
// 8th part, then the 8 row sums in order (a fixed order: deterministic).
__global__ __launch_bounds__(256) void parts_reduce_kernel(const float* __restrict__ part,
                                                           int nparts, int n,
                                                           float* __restrict__ out) {
  __shared__ float red[8][33];
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
  const int c = blockIdx.x * 32 + tx;
  float s = 0.f;
  if (c < n) {  // parts ty, ty + 8, … in order, eight loads in flight at a time
    int p = ty;
    for (; p + 56 < nparts; p += 64) {
      float v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = part[static_cast<long long>(p + 8 * u) * n + c];
#pragma unroll
      for (int u = 0; u < 8; ++u) s += v[u];
    }
    for (; p < nparts; p += 8) s += part[static_cast<long long>(p) * n + c];
  }
  red[ty][tx] = s;
  __syncthreads();
  if (ty == 0 && c < n) {
    float t = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) t += red[i][tx];
    out[c] += t;
  }
}

// ---------------------------------------------------------------- column sums
constexpr int kColRows = 64;

// part[p][c] = Σ a[r][c] over the kColRows rows of part p. A workgroup takes 32·VEC columns
// (VEC per 16-byte load) and 8 row lanes: lane ty sums rows r0 + ty, r0 + ty + 8, … (all
// its loads in flight at once), and the 8 lane sums are added in order through LDS — a
// fixed order, so the result is deterministic. Columns are grouped VEC at a time when n
// and the row stride allow 16-byte loads (colsum_vec), else one at a time.
template <typename T, int VEC>
__global__ __launch_bounds__(256) void colsum_part_kernel(const T* __restrict__ a,
                                                          long long lda, int rows, int n,
                                                          float* __restrict__ part) {
  constexpr int RL = 8, PER = kColRows / RL;
  __shared__ float red[RL][32 * VEC + 1];
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
  const int c0 = blockIdx.x * 32 * VEC + tx * VEC;
  const int r0 = blockIdx.y * kColRows;
  float s[VEC];
#pragma unroll
  for (int e = 0; e < VEC; ++e) s[e] = 0.f;
  if (c0 < n) {
    T v[PER][VEC];
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int r = r0 + ty + RL * j;
      const T* src = a + static_cast<long long>(r < rows ? r : 0) * lda + c0;
      if constexpr (VEC == 1) {
        v[j][0] = r < rows ? src[0] : static_cast<T>(0.f);
      } else {
        typedef T vec_t __attribute__((ext_vector_type(VEC)));
        const vec_t w = *reinterpret_cast<const vec_t*>(src);
#pragma unroll
        for (int e = 0; e < VEC; ++e) v[j][e] = r < rows ? w[e] : static_cast<T>(0.f);
      }
    }
#pragma unroll
    for (int j = 0; j < PER; ++j)
#pragma unroll
      for (int e = 0; e < VEC; ++e) s[e] += static_cast<float>(v[j][e]);
  }
#pragma unroll
  for (int e = 0; e < VEC; ++e) red[ty][tx * VEC + e] = s[e];
  __syncthreads();
  for (int i = threadIdx.x; i < 32 * VEC; i += 256) {
    const int c = blockIdx.x * 32 * VEC + i;
    if (c >= n) continue;
    float t = 0.f;
#pragma unroll
    for (int l = 0; l < RL; ++l) t += red[l][i];
    part[static_cast<long long>(blockIdx.y) * n + c] = t;
  }
}

// -------------------------------------------------------- cross-entropy backward
// One block per row: probs = exp(l − max)·(1/Σexp), probs[label] −= 1, × scale. fp16: the
// shift, exp and products rounded to fp16, Σexp in fp32 and 1/Σexp and scale cast to fp16
// (kernels/fused_crossentropy.py:41-49 with the forward's fp32 sum, :20-24).
template <typename T>
__global__ __launch_bounds__(256) void ce_grad_kernel(T* __restrict__ lg, int V,
                                                      const int64_t* __restrict__ labels,
                                                      long long ignore_index, int has_ignore,
                                                      float scale) {
#pragma clang fp contract(off)
  __shared__ float red[4];
  T* p = lg + static_cast<long long>(blockIdx.x) * V;
  const long long label = labels[blockIdx.x];
  if (has_ignore && label == ignore_index) {
    for (int i = threadIdx.x; i < V; i += 256) p[i] = static_cast<T>(0.f);
    return;
  }
  float mx = -INFINITY;
  for (int i = threadIdx.x; i < V; i += 256) mx = fmaxf(mx, static_cast<float>(p[i]));
  mx = wave_max(mx);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  float se = 0.f;
  for (int i = threadIdx.x; i < V; i += 256) se += rnd<T>(expf(rnd<T>(static_cast<float>(p[i]) - mx)));
  se = block_sum(se, red);
  const float inv = rnd<T>(1.0f / se);
  const float sc = rnd<T>(scale);
  for (int i = threadIdx.x; i < V; i += 256) {
    float v = rnd<T>(rnd<T>(expf(rnd<T>(static_cast<float>(p[i]) - mx))) * inv);
    if (i == label) v = rnd<T>(v - 1.0f);
    p[i] = static_cast<T>(v * sc);
  }
}

// The same arithmetic with the row held in registers (one HBM read and one write per
// element instead of three reads): thread t owns the 16-byte chunks t, t + 256, … of the
// row (NCH of them at most); V a multiple of the chunk's element count. The partial sums
// of Σexp run over a different element order than ce_grad_kernel's.
template <typename T, int NCH>
__global__ __launch_bounds__(256) void ce_grad_reg_kernel(T* __restrict__ lg, int V,
                                                          const int64_t* __restrict__ labels,
                                                          long long ignore_index, int has_ignore,
                                                          float scale) {
#pragma clang fp contract(off)
  constexpr int E = 16 / static_cast<int>(sizeof(T));
  typedef T vec_t __attribute__((ext_vector_type(E)));
  __shared__ float red[4];
  vec_t* p = reinterpret_cast<vec_t*>(lg + static_cast<long long>(blockIdx.x) * V);
  const int nch = V / E, tid = threadIdx.x;
  const long long label = labels[blockIdx.x];
  if (has_ignore && label == ignore_index) {
    vec_t z;
#pragma unroll
    for (int e = 0; e < E; ++e) z[e] = static_cast<T>(0.f);
    for (int c = tid; c < nch; c += 256) p[c] = z;
    return;
  }
  vec_t r[NCH];
  float mx = -INFINITY;
#pragma unroll
  for (int k = 0; k < NCH; ++k) {
    const int c = tid + 256 * k;
    if (c < nch) {
      r[k] = p[c];
#pragma unroll
      for (int e = 0; e < E; ++e) mx = fmaxf(mx, static_cast<float>(r[k][e]));
    }
  }
  mx = wave_max(mx);
  if ((tid & 63) == 0) red[tid >> 6] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  float se = 0.f;
#pragma unroll
  for (int k = 0; k < NCH; ++k)
    if (tid + 256 * k < nch) {
#pragma unroll
      for (int e = 0; e < E; ++e) se += rnd<T>(expf(rnd<T>(static_cast<float>(r[k][e]) - mx)));
    }
  se = block_sum(se, red);
  const float inv = rnd<T>(1.0f / se);
  const float sc = rnd<T>(scale);
#pragma unroll
  for (int k = 0; k < NCH; ++k) {
    const int c = tid + 256 * k;
    if (c < nch) {
      vec_t o;
#pragma unroll
      for (int e = 0; e < E; ++e) {
        float v = rnd<T>(rnd<T>(expf(rnd<T>(static_cast<float>(r[k][e]) - mx))) * inv);
        if (c * E + e == label) v = rnd<T>(v - 1.0f);
        o[e] = static_cast<T>(v * sc);
      }
      p[c] = o;
    }
  }
}

// ------------------------------------------------------------ attention backward
// dvec[(b·H + h)·S + s] = Σ_c dout·o over the head's columns (= Σ_j P·dP of the
// softmax backward, kernels/fused_sdpa.py:26-29).
template <typename T>
__global__ __launch_bounds__(256) void attn_bwd_dot_kernel(AttnBwdArgs a) {
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int R = a.B * a.S;
  if (t >= R * a.H) return;
  const int r = t / a.H, h = t - (t / a.H) * a.H;
  const int b = r / a.S, s = r - (r / a.S) * a.S;
  const long long off = static_cast<long long>(r) * a.H * a.dk + h * a.dk;
  float v = 0.f;
  const T* dout = static_cast<const T*>(a.dout);
  const T* o = static_cast<const T*>(a.o);
  for (int c = lane; c < a.dk; c += 64) v += static_cast<float>(dout[off + c]) * static_cast<float>(o[off + c]);
  v = wave_sum(v);
  if (lane == 0) a.dvec[(static_cast<long long>(b) * a.H + h) * a.S + s] = v;
}

// The forward's score of q·k: q·k·(1/scale) in fp32; fp16 rnd(rnd(q·k)·(1/fp16(scale))),
// the rounding of the fp16 prefill kernel.
template <typename T>
__device__ __forceinline__ float attn_score(float dot, float mul) {
  if constexpr (sizeof(T) == 4) return dot * mul;
  else return rnd<T>(rnd<T>(dot) * mul);
}
template <typename T>
__device__ __forceinline__ float score_mul(float scale) {
  if constexpr (sizeof(T) == 4) return 1.0f / scale;
  else return 1.0f / static_cast<float>(static_cast<T>(scale));
}

// Shared per-tile step: thread t scores EPT (query i, key j) pairs of a BT × BT tile,
// i = t / TPR, j = (t % TPR)·EPT + e: p = exp(q·k/scale − lse_i) where key ≤ query (both
// inside the sequence), else 0; ds = p·(dO_i·v_j − D_i)/scale. A full (non-causal) call
// scores every key inside the sequence with the non-causal forward's roundings
// (rnd(rnd(q·k) / scale), then + mask[query][key] rounded) — a masked −inf gives p = 0.
template <int DK, int BT, typename T>
struct AttnTile {
  static constexpr int EPT = BT * BT / 256;
  static constexpr int TPR = BT / EPT;
  float Qs[BT][DK + 1];
  float dOs[BT][DK + 1];
  float Ks[BT][DK + 1];
  float Vs[BT][DK + 1];
  float Ps[BT][BT + 1];
  float dSs[BT][BT + 1];
  float lse[BT];
  float D[BT];

  __device__ void scores(int q_lo, int k_lo, int S, float scale, int full, const T* mask) {
    const float mul = score_mul<T>(scale), inv_scale = 1.0f / scale;
    const float scale_t = static_cast<float>(static_cast<T>(scale));
    const int t = threadIdx.x;
    const int i = t / TPR, j0 = (t % TPR) * EPT;
    const int qi = q_lo + i;
#pragma unroll
    for (int e = 0; e < EPT; ++e) {
      const int j = j0 + e, kj = k_lo + j;
      float p = 0.f, ds = 0.f;
      if (qi < S && (full ? kj < S : kj <= qi)) {
        float dot = 0.f, dp = 0.f;
#pragma unroll 8
        for (int c = 0; c < DK; ++c) {
          dot += Qs[i][c] * Ks[j][c];
          dp += dOs[i][c] * Vs[j][c];
        }
        float sc;
        if (full) {
          sc = rnd<T>(rnd<T>(dot) / scale_t);
          if (mask) sc = rnd<T>(sc + static_cast<float>(mask[static_cast<long long>(qi) * S + kj]));
        } else {
          sc = attn_score<T>(dot, mul);
        }
        p = sc == -INFINITY ? 0.f : expf(sc - lse[i]);
        ds = p * (dp - D[i]) * inv_scale;
      }
      Ps[i][j] = p;
      dSs[i][j] = ds;
    }
  }
};

// rows [lo, lo + BT) of a head-major (B·H, S, dk) tensor into dst (0 past S and in the
// padding columns dk ≤ c < DK)
template <int DK, int BT, typename T>
__device__ __forceinline__ void load_rows(float (*dst)[DK + 1], const T* __restrict__ src,
                                          int lo, int S, int dk) {
  for (int e = threadIdx.x; e < BT * DK; e += 256) {
    const int r = e / DK, c = e - (e / DK) * DK;
    dst[r][c] = lo + r < S && c < dk ? static_cast<float>(src[static_cast<long long>(lo + r) * dk + c]) : 0.f;
  }
}

// rows [lo, lo + BT) of head h of a merged (B·S, H·dk) tensor
template <int DK, int BT, typename T>
__device__ __forceinline__ void load_merged(float (*dst)[DK + 1], const T* __restrict__ src,
                                            int b, int h, int H, int lo, int S, int dk) {
  for (int e = threadIdx.x; e < BT * DK; e += 256) {
    const int r = e / DK, c = e - (e / DK) * DK;
    dst[r][c] = lo + r < S && c < dk
                    ? static_cast<float>(src[(static_cast<long long>(b) * S + lo + r) * H * dk + h * dk + c])
                    : 0.f;
  }
}

// The scalar kernels keep their tiles in dynamic LDS (at DK 256 they exceed the 64 KiB
// of static shared memory). DK is the padded tile width; the runtime a.dk ≤ DK is the
// head dim (columns dk ≤ c < DK hold zeros and are never written back).
extern __shared__ __align__(16) unsigned char attn_bwd_smem[];

// dK, dV of BT keys: walk the query tiles from the key tile on (causal; every query tile
// when full).
template <int DK, int BT, typename T>
__global__ __launch_bounds__(256) void attn_bwd_dkdv_kernel(AttnBwdArgs a) {
  AttnTile<DK, BT, T>& sh = *reinterpret_cast<AttnTile<DK, BT, T>*>(attn_bwd_smem);
  const T* qg = static_cast<const T*>(a.q);
  const T* kg = static_cast<const T*>(a.k);
  const T* vg = static_cast<const T*>(a.v);
  const T* og = static_cast<const T*>(a.dout);
  constexpr int TPK = 256 / BT;       // threads per key row of the output
  constexpr int NCOL = (DK + TPK - 1) / TPK;
  const int bh = blockIdx.y, b = bh / a.H, h = bh - (bh / a.H) * a.H;
  const int S = a.S, k_lo = blockIdx.x * BT, hd = a.dk;
  const long long hoff = static_cast<long long>(bh) * S * hd;
  load_rows<DK, BT>(sh.Ks, kg + hoff, k_lo, S, hd);
  load_rows<DK, BT>(sh.Vs, vg + hoff, k_lo, S, hd);
  const int jo = threadIdx.x / TPK, co = threadIdx.x % TPK;
  float dk[NCOL], dv[NCOL];
#pragma unroll
  for (int u = 0; u < NCOL; ++u) dk[u] = dv[u] = 0.f;
  const T* mask = static_cast<const T*>(a.mask);
  for (int q_lo = a.full ? 0 : k_lo; q_lo < S; q_lo += BT) {
    __syncthreads();  // the previous tile's readers are done
    load_rows<DK, BT>(sh.Qs, qg + hoff, q_lo, S, hd);
    load_merged<DK, BT>(sh.dOs, og, b, h, a.H, q_lo, S, hd);
    for (int i = threadIdx.x; i < BT; i += 256) {
      const bool ok = q_lo + i < S;
      sh.lse[i] = ok ? a.lse[static_cast<long long>(bh) * S + q_lo + i] : 0.f;
      sh.D[i] = ok ? a.dvec[static_cast<long long>(bh) * S + q_lo + i] : 0.f;
    }
    __syncthreads();
    sh.scores(q_lo, k_lo, S, a.scale, a.full, mask);
    __syncthreads();
#pragma unroll
    for (int u = 0; u < NCOL; ++u) {
      const int c = co + TPK * u;
      if (c < DK) {
        float sv = 0.f, sk = 0.f;
#pragma unroll 8
        for (int i = 0; i < BT; ++i) {
          sv += sh.Ps[i][jo] * sh.dOs[i][c];
          sk += sh.dSs[i][jo] * sh.Qs[i][c];
        }
        dv[u] += sv;
        dk[u] += sk;
      }
    }
  }
  const int key = k_lo + jo;
  if (key < S) {
    const int d = a.H * hd;
    T* row = static_cast<T*>(a.dqkv) + (static_cast<long long>(b) * S + key) * 3 * d + h * hd;
#pragma unroll
    for (int u = 0; u < NCOL; ++u) {
      const int c = co + TPK * u;
      if (c < hd) {
        row[d + c] = static_cast<T>(dk[u]);
        row[2 * d + c] = static_cast<T>(dv[u]);
      }
    }
  }
}

// dQ of BT queries: walk the key tiles up to the query tile (causal; every key tile when
// full).
template <int DK, int BT, typename T>
__global__ __launch_bounds__(256) void attn_bwd_dq_kernel(AttnBwdArgs a) {
  AttnTile<DK, BT, T>& sh = *reinterpret_cast<AttnTile<DK, BT, T>*>(attn_bwd_smem);
  const T* qg = static_cast<const T*>(a.q);
  const T* kg = static_cast<const T*>(a.k);
  const T* vg = static_cast<const T*>(a.v);
  const T* og = static_cast<const T*>(a.dout);
  constexpr int TPK = 256 / BT;
  constexpr int NCOL = (DK + TPK - 1) / TPK;
  const int bh = blockIdx.y, b = bh / a.H, h = bh - (bh / a.H) * a.H;
  const int S = a.S, q_lo = blockIdx.x * BT, hd = a.dk;
  const long long hoff = static_cast<long long>(bh) * S * hd;
  load_rows<DK, BT>(sh.Qs, qg + hoff, q_lo, S, hd);
  load_merged<DK, BT>(sh.dOs, og, b, h, a.H, q_lo, S, hd);
  for (int i = threadIdx.x; i < BT; i += 256) {
    const bool ok = q_lo + i < S;
    sh.lse[i] = ok ? a.lse[static_cast<long long>(bh) * S + q_lo + i] : 0.f;
    sh.D[i] = ok ? a.dvec[static_cast<long long>(bh) * S + q_lo + i] : 0.f;
  }
  const int io = threadIdx.x / TPK, co = threadIdx.x % TPK;
  float dq[NCOL];
#pragma unroll
  for (int u = 0; u < NCOL; ++u) dq[u] = 0.f;
  const int k_end = a.full ? S : min(S, q_lo + BT);
  const T* mask = static_cast<const T*>(a.mask);
  for (int k_lo = 0; k_lo < k_end; k_lo += BT) {
    __syncthreads();
    load_rows<DK, BT>(sh.Ks, kg + hoff, k_lo, S, hd);
    load_rows<DK, BT>(sh.Vs, vg + hoff, k_lo, S, hd);
    __syncthreads();
    sh.scores(q_lo, k_lo, S, a.scale, a.full, mask);
    __syncthreads();
#pragma unroll
    for (int u = 0; u < NCOL; ++u) {
      const int c = co + TPK * u;
      if (c < DK) {
        float s = 0.f;
#pragma unroll 8
        for (int j = 0; j < BT; ++j) s += sh.dSs[io][j] * sh.Ks[j][c];
        dq[u] += s;
      }
    }
  }
  const int q = q_lo + io;
  if (q < S) {
    const int d = a.H * hd;
    T* row = static_cast<T*>(a.dqkv) + (static_cast<long long>(b) * S + q) * 3 * d + h * hd;
#pragma unroll
    for (int u = 0; u < NCOL; ++u) {
      const int c = co + TPK * u;
      if (c < hd) row[c] = static_cast<T>(dq[u]);
    }
  }
}

// ---- MFMA variant (head dims 64 and 128): 64 keys × 64 queries per step, 4 waves.
// Wave w = (wq, wk) = (w / 2, w % 2) takes the 32 × 32 sub-tile of queries 32·wq… and keys
// 32·wk…; MFMA 32×32×2 fp32 throughout. A 32 × 32 result tile in registers holds, in
// lane l and register r, row 8(r/4) + 4(l/32) + r%4 and column l%32; the products that
// reduce over that row index take the registers themselves as their A operand (lane l
// supplies rows f(r) for k = 0 and f(r) + 4 for k = 1, which only reorders the sum), so
// P and dS never go through LDS. Tiles in LDS are [row][DK + 1] fp32.
constexpr int kAT = 64;

// Grid (tiles, B·H) of the attention backward: when B·H is a multiple of 8, every tile of
// one (row, head) runs on one XCD (workgroups are dealt to the 8 XCDs round robin in
// dispatch order), so the Q / dO (or K / V) rows its tiles share come from that XCD's L2
// instead of being fetched by all eight; tiles of a (row, head) run in index order.
__device__ __forceinline__ void bwd_tile_order(int& bh, int& t) {
  bh = blockIdx.y;
  t = blockIdx.x;
  if (gridDim.y % 8 == 0) {
    const int n = blockIdx.x + blockIdx.y * gridDim.x;
    const int slot = n >> 3;
    bh = (n & 7) + 8 * (slot / gridDim.x);
    t = slot % gridDim.x;
  }
}
constexpr float kLog2eF = 1.4426950408889634f;

template <int DK>
constexpr size_t attn_mfma_lds() {
  return (4 * kAT * (DK + 1) + 2 * kAT) * sizeof(float);
}

// rows [lo, lo + 64) of a head-major (S, DK) slice into a [64][DK + 1] tile (0 past S)
template <int DK, typename T>
__device__ __forceinline__ void tile_rows(float* dst, const T* __restrict__ src, int lo, int S) {
  for (int e = threadIdx.x; e < kAT * DK / 4; e += 256) {
    const int r = e / (DK / 4), c = (e - r * (DK / 4)) * 4;
    floatx4 v = {0.f, 0.f, 0.f, 0.f};
    if (lo + r < S) v = ld4(src + static_cast<long long>(lo + r) * DK + c);
#pragma unroll
    for (int j = 0; j < 4; ++j) dst[r * (DK + 1) + c + j] = v[j];
  }
}

// rows [lo, lo + 64) of head h of a merged (B·S, H·DK) tensor
template <int DK, typename T>
__device__ __forceinline__ void tile_merged(float* dst, const T* __restrict__ src, int b, int h,
                                            int H, int lo, int S) {
  for (int e = threadIdx.x; e < kAT * DK / 4; e += 256) {
    const int r = e / (DK / 4), c = (e - r * (DK / 4)) * 4;
    floatx4 v = {0.f, 0.f, 0.f, 0.f};
    if (lo + r < S) v = ld4(src + (static_cast<long long>(b) * S + lo + r) * H * DK + h * DK + c);
#pragma unroll
    for (int j = 0; j < 4; ++j) dst[r * (DK + 1) + c + j] = v[j];
  }
}

__device__ __forceinline__ int d_row(int r, int lane) { return 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3); }

// A 64 × DK tile staged through registers (DK/16 16-byte vectors per thread) so that the
// next tile's loads are in flight while the current one multiplies.
template <int DK, typename T>
struct TileRegs {
  floatx4 v[DK / 16];
  // rows [lo, lo + 64) of a row-major source with row stride ld (0 past S)
  __device__ __forceinline__ void load(const T* __restrict__ src, long long ld, int lo, int S) {
#pragma unroll
    for (int i = 0; i < DK / 16; ++i) {
      const int e = threadIdx.x + 256 * i;
      const int r = e / (DK / 4), c = (e - r * (DK / 4)) * 4;
      const floatx4 z = {0.f, 0.f, 0.f, 0.f};
      v[i] = lo + r < S ? ld4(src + static_cast<long long>(lo + r) * ld + c) : z;
    }
  }
  __device__ __forceinline__ void store(float* dst) const {
#pragma unroll
    for (int i = 0; i < DK / 16; ++i) {
      const int e = threadIdx.x + 256 * i;
      const int r = e / (DK / 4), c = (e - r * (DK / 4)) * 4;
#pragma unroll
      for (int j = 0; j < 4; ++j) dst[r * (DK + 1) + c + j] = v[i][j];
    }
  }
};

// dK, dV of 64 keys; the query tiles from the key tile on.
template <int DK, typename T>
__global__ __launch_bounds__(256, 2) void attn_bwd_dkdv_mfma(AttnBwdArgs a) {
  extern __shared__ float lds[];
  constexpr int P = DK + 1, NJ = DK / 32;
  float* Ks = lds;
  float* Vs = Ks + kAT * P;
  float* Qs = Vs + kAT * P;
  float* Os = Qs + kAT * P;
  float* Ls = Os + kAT * P;
  float* Ds = Ls + kAT;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, wq = w >> 1, wk = w & 1;
  const int l32 = lane & 31, hi = lane >> 5;
  int bh, t;
  bwd_tile_order(bh, t);
  const int b = bh / a.H, h = bh - (bh / a.H) * a.H;
  const int S = a.S, k_lo = t * kAT;  // the longest key tiles (most query tiles) first
  const long long hoff = static_cast<long long>(bh) * S * DK;
  tile_rows<DK>(Ks, static_cast<const T*>(a.k) + hoff, k_lo, S);
  tile_rows<DK>(Vs, static_cast<const T*>(a.v) + hoff, k_lo, S);
  floatx16 dv[NJ], dk[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) dv[j][r] = dk[j][r] = 0.f;
  const int key = k_lo + 32 * wk + l32;  // this lane's key (column of S)
  const float inv_scale = 1.0f / a.scale, mul = score_mul<T>(a.scale);
  const T* dout_b = static_cast<const T*>(a.dout) + static_cast<long long>(b) * S * a.H * DK + h * DK;
  const T* qg = static_cast<const T*>(a.q);
  TileRegs<DK, T> nq, no;
  float nl = 0.f, nd = 0.f;
  auto fetch = [&](int lo) {
    nq.load(qg + hoff, DK, lo, S);
    no.load(dout_b, static_cast<long long>(a.H) * DK, lo, S);
    if (threadIdx.x < kAT) {
      const int q = lo + threadIdx.x;
      nl = q < S ? a.lse[static_cast<long long>(bh) * S + q] : 0.f;
      nd = q < S ? a.dvec[static_cast<long long>(bh) * S + q] : 0.f;
    }
  };
  fetch(k_lo);
  for (int q_lo = k_lo; q_lo < S; q_lo += kAT) {
    __syncthreads();  // every wave is done with the previous tile
    nq.store(Qs);
    no.store(Os);
    if (threadIdx.x < kAT) {
      Ls[threadIdx.x] = nl;
      Ds[threadIdx.x] = nd;
    }
    __syncthreads();
    if (q_lo + kAT < S) fetch(q_lo + kAT);
    floatx16 sc, dp;
#pragma unroll
    for (int r = 0; r < 16; ++r) sc[r] = dp[r] = 0.f;
    const float* qa = Qs + (32 * wq + l32) * P + hi;
    const float* oa = Os + (32 * wq + l32) * P + hi;
    const float* kb = Ks + (32 * wk + l32) * P + hi;
    const float* vb = Vs + (32 * wk + l32) * P + hi;
#pragma unroll 8
    for (int c0 = 0; c0 < DK; c0 += 2) {
      sc = __builtin_amdgcn_mfma_f32_32x32x2f32(qa[c0], kb[c0], sc, 0, 0, 0);
      dp = __builtin_amdgcn_mfma_f32_32x32x2f32(oa[c0], vb[c0], dp, 0, 0, 0);
    }
    // the lane's 16 query rows' statistics as broadcast 16-byte reads; p = exp(s − lse) as
    // exp2(s·log₂e − lse·log₂e); the mask only on the first and a ragged last tile
    float nl2[16], dd[16];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const floatx4 l4 = *reinterpret_cast<const floatx4*>(Ls + 32 * wq + 8 * g + 4 * hi);
      const floatx4 d4 = *reinterpret_cast<const floatx4*>(Ds + 32 * wq + 8 * g + 4 * hi);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        nl2[4 * g + e] = -l4[e] * kLog2eF;
        dd[4 * g + e] = d4[e];
      }
    }
    if (q_lo < k_lo + kAT || q_lo + kAT > S) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int q = q_lo + 32 * wq + d_row(r, lane);
        float p = 0.f;
        if (key <= q && q < S)
          p = __builtin_amdgcn_exp2f(__builtin_fmaf(attn_score<T>(sc[r], mul), kLog2eF, nl2[r]));
        sc[r] = p;
        dp[r] = p * (dp[r] - dd[r]) * inv_scale;
      }
    } else {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(attn_score<T>(sc[r], mul), kLog2eF, nl2[r]));
        sc[r] = p;
        dp[r] = p * (dp[r] - dd[r]) * inv_scale;
      }
    }
    // dV[key][c] += Σ_q P[q][key]·dO[q][c];  dK[key][c] += Σ_q dS[q][key]·Q[q][c]
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int ql = 32 * wq + d_row(r, lane);
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        dv[j] = __builtin_amdgcn_mfma_f32_32x32x2f32(sc[r], Os[ql * P + 32 * j + l32], dv[j], 0, 0, 0);
        dk[j] = __builtin_amdgcn_mfma_f32_32x32x2f32(dp[r], Qs[ql * P + 32 * j + l32], dk[j], 0, 0, 0);
      }
    }
  }
  // the two query halves (wq = 0, 1) of each key half meet in LDS
  __syncthreads();
  float* red = Qs;  // 2 key halves × (dv, dk) × NJ × 16 × 64 floats
  if (wq == 1) {
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        red[(((wk * 2 + 0) * NJ + j) * 16 + r) * 64 + lane] = dv[j][r];
        red[(((wk * 2 + 1) * NJ + j) * 16 + r) * 64 + lane] = dk[j][r];
      }
  }
  __syncthreads();
  if (wq == 0) {
    const int d = a.H * DK;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int kk = k_lo + 32 * wk + d_row(r, lane);
      if (kk < S) {
        T* row = static_cast<T*>(a.dqkv) + (static_cast<long long>(b) * S + kk) * 3 * d + h * DK;
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
          row[d + 32 * j + l32] = static_cast<T>(dk[j][r] + red[(((wk * 2 + 1) * NJ + j) * 16 + r) * 64 + lane]);
          row[2 * d + 32 * j + l32] = static_cast<T>(dv[j][r] + red[(((wk * 2 + 0) * NJ + j) * 16 + r) * 64 + lane]);
        }
      }
    }
  }
}

// dQ of 64 queries; the key tiles up to the query tile. Wave w = (wk, wq) = (w / 2, w % 2)
// computes Sᵀ (keys as rows) so that its registers feed dQ = dS·K as the A operand.
template <int DK, typename T>
__global__ __launch_bounds__(256) void attn_bwd_dq_mfma(AttnBwdArgs a) {
  extern __shared__ float lds[];
  constexpr int P = DK + 1, NJ = DK / 32;
  float* Ks = lds;
  float* Vs = Ks + kAT * P;
  float* Qs = Vs + kAT * P;
  float* Os = Qs + kAT * P;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, wk = w >> 1, wq = w & 1;
  const int l32 = lane & 31, hi = lane >> 5;
  int bh, t;
  bwd_tile_order(bh, t);
  const int b = bh / a.H, h = bh - (bh / a.H) * a.H;
  const int S = a.S, q_lo = (gridDim.x - 1 - t) * kAT;  // the longest query tiles first
  const long long hoff = static_cast<long long>(bh) * S * DK;
  const T* kg = static_cast<const T*>(a.k);
  const T* vg = static_cast<const T*>(a.v);
  tile_rows<DK>(Qs, static_cast<const T*>(a.q) + hoff, q_lo, S);
  tile_merged<DK>(Os, static_cast<const T*>(a.dout), b, h, a.H, q_lo, S);
  const int q = q_lo + 32 * wq + l32;  // this lane's query (column of Sᵀ)
  const float lse = q < S ? a.lse[static_cast<long long>(bh) * S + q] : 0.f;
  const float dd = q < S ? a.dvec[static_cast<long long>(bh) * S + q] : 0.f;
  floatx16 dq[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) dq[j][r] = 0.f;
  const int k_end = min(S, q_lo + kAT);
  const float inv_scale = 1.0f / a.scale, mul = score_mul<T>(a.scale);
  TileRegs<DK, T> nk, nv;
  nk.load(kg + hoff, DK, 0, S);
  nv.load(vg + hoff, DK, 0, S);
  for (int k_lo = 0; k_lo < k_end; k_lo += kAT) {
    __syncthreads();  // every wave is done with the previous tile
    nk.store(Ks);
    nv.store(Vs);
    __syncthreads();
    if (k_lo + kAT < k_end) {
      nk.load(kg + hoff, DK, k_lo + kAT, S);
      nv.load(vg + hoff, DK, k_lo + kAT, S);
    }
    floatx16 sc, dp;
#pragma unroll
    for (int r = 0; r < 16; ++r) sc[r] = dp[r] = 0.f;
    const float* ka = Ks + (32 * wk + l32) * P + hi;
    const float* va = Vs + (32 * wk + l32) * P + hi;
    const float* qb = Qs + (32 * wq + l32) * P + hi;
    const float* ob = Os + (32 * wq + l32) * P + hi;
#pragma unroll 8
    for (int c0 = 0; c0 < DK; c0 += 2) {
      sc = __builtin_amdgcn_mfma_f32_32x32x2f32(ka[c0], qb[c0], sc, 0, 0, 0);
      dp = __builtin_amdgcn_mfma_f32_32x32x2f32(va[c0], ob[c0], dp, 0, 0, 0);
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int kk = k_lo + 32 * wk + d_row(r, lane);
      float p = 0.f;
      if (kk <= q && q < S)
        p = __builtin_amdgcn_exp2f(__builtin_fmaf(attn_score<T>(sc[r], mul), kLog2eF, -lse * kLog2eF));
      dp[r] = p * (dp[r] - dd) * inv_scale;
    }
    // dQ[q][c] += Σ_key dS[q][key]·K[key][c]
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int kl = 32 * wk + d_row(r, lane);
#pragma unroll
      for (int j = 0; j < NJ; ++j)
        dq[j] = __builtin_amdgcn_mfma_f32_32x32x2f32(dp[r], Ks[kl * P + 32 * j + l32], dq[j], 0, 0, 0);
    }
  }
  __syncthreads();
  float* red = Ks;  // 2 query halves × NJ × 16 × 64 floats
  if (wk == 1) {
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) red[((wq * NJ + j) * 16 + r) * 64 + lane] = dq[j][r];
  }
  __syncthreads();
  if (wk == 0) {
    const int d = a.H * DK;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int qq = q_lo + 32 * wq + d_row(r, lane);
      if (qq < S) {
        T* row = static_cast<T*>(a.dqkv) + (static_cast<long long>(b) * S + qq) * 3 * d + h * DK;
#pragma unroll
        for (int j = 0; j < NJ; ++j)
          row[32 * j + l32] = static_cast<T>(dq[j][r] + red[((wq * NJ + j) * 16 + r) * 64 + lane]);
      }
    }
  }
}

// ---- fp16 models on the fp16 MFMA (32×32×16, head dims 64 and 128): the same two kernels
// and wave layout as above with fp16 tiles in LDS — [row][dim] for the products that reduce
// over the head dimension, and a transposed [dim][row] copy of the operand that the
// P / dS products reduce over by rows (Q and dO in the dK/dV kernel, K in the dQ kernel).
// P and dS are rounded to fp16 where they enter the MFMA (the reference's fp16 backward
// holds them in fp16). A 16-row step of those products takes rows f(r) (k slots 0–7) and
// f(r) + 4 (slots 8–15) from registers r = 8s … 8s + 7, i.e. rows 16s + {0–3, 8–11} and
// 16s + {4–7, 12–15}: two 8-byte reads of the transposed copy per fragment.
// The transposed copies' rows are 34 dwords apart: the 32 rows an 8-byte fragment read
// takes (lanes 0-31, and 32-63) then fall on 32 distinct bank pairs (36 dwords put rows l
// and l + 16 on one pair: half of all LDS cycles of the two kernels were bank conflicts).
constexpr int kATT = kAT + 4;
template <int DK>
constexpr size_t attn_f16_lds() {
  return (static_cast<size_t>(4) * kAT * (DK + 8) + 2 * DK * kATT) * sizeof(half_t) +
         2 * kAT * sizeof(float);
}

// rows [lo, lo + 64) of a (row stride ld) fp16 source: natural [row][DK + 8] copy into X
// and, when XT is given, the transposed [dim][64 + 8] copy, in blocks of 4 rows × 8 dims
// (block b of 16·DK/8: rows 4·(b / (DK/8)) …, dims 8·(b % (DK/8)) …) taken by threads
// first … first + 16·DK/8 − 1.
// fetch16 loads the block into registers, put16 writes it (and its transpose) to LDS;
// stage16 does both.
template <int DK>
__device__ __forceinline__ void fetch16(half8 (&v)[4], const half_t* __restrict__ src, long long ld,
                                        int lo, int S, int first) {
  constexpr int NB = 16 * DK / 8;
  const int b = static_cast<int>(threadIdx.x) - first;
  if (b < 0 || b >= NB) return;
  const int r0 = 4 * (b / (DK / 8)), c = 8 * (b % (DK / 8));
  const half8 z = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
  for (int i = 0; i < 4; ++i)
    v[i] = lo + r0 + i < S ? *reinterpret_cast<const half8*>(src + static_cast<long long>(lo + r0 + i) * ld + c) : z;
}

template <int DK>
__device__ __forceinline__ void put16(half_t* X, half_t* XT, const half8 (&v)[4], int first) {
  constexpr int PA = DK + 8, PT = kATT, NB = 16 * DK / 8;
  const int b = static_cast<int>(threadIdx.x) - first;
  if (b < 0 || b >= NB) return;
  const int r0 = 4 * (b / (DK / 8)), c = 8 * (b % (DK / 8));
#pragma unroll
  for (int i = 0; i < 4; ++i) *reinterpret_cast<half8*>(X + (r0 + i) * PA + c) = v[i];
  if (XT) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const half4 w = {v[0][j], v[1][j], v[2][j], v[3][j]};
      *reinterpret_cast<half4*>(XT + (c + j) * PT + r0) = w;
    }
  }
}

template <int DK>
__device__ __forceinline__ void stage16(half_t* X, half_t* XT, const half_t* __restrict__ src, long long ld,
                                        int lo, int S, int first) {
  half8 v[4];
  fetch16<DK>(v, src, ld, lo, S, first);
  put16<DK>(X, XT, v, first);
}

// A 16-row fragment of a transposed [dim][64 + 8] tile: dims d0 + l % 32, rows of step s
// within the 32-row block rb as the register layout pairs them.
__device__ __forceinline__ half8 frag_t(const half_t* XT, int d0, int rb, int s, int lane) {
  constexpr int PT = kATT;
  const half_t* p = XT + (d0 + (lane & 31)) * PT + rb + 16 * s + 4 * (lane >> 5);
  const half4 lo = *reinterpret_cast<const half4*>(p);
  const half4 hi = *reinterpret_cast<const half4*>(p + 8);
  const half8 f = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  return f;
}

__device__ __forceinline__ half8 regs16(const floatx16& v, int s) {
  half8 f;
#pragma unroll
  for (int j = 0; j < 8; ++j) f[j] = static_cast<half_t>(v[8 * s + j]);
  return f;
}

template <int DK>
__global__ __launch_bounds__(256, 2) void attn_bwd_dkdv_f16(AttnBwdArgs a) {
  extern __shared__ __attribute__((aligned(16))) half_t lds16[];
  constexpr int PA = DK + 8, PT = kATT, NJ = DK / 32;
  half_t* Ks = lds16;
  half_t* Vs = Ks + kAT * PA;
  half_t* Qs = Vs + kAT * PA;
  half_t* Os = Qs + kAT * PA;
  half_t* QT = Os + kAT * PA;
  half_t* OT = QT + DK * PT;
  float* Ls = reinterpret_cast<float*>(OT + DK * PT);
  float* Ds = Ls + kAT;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, wq = w >> 1, wk = w & 1;
  const int l32 = lane & 31, hi = lane >> 5;
  int bh, t;
  bwd_tile_order(bh, t);
  const int b = bh / a.H, h = bh - (bh / a.H) * a.H;
  const int S = a.S, k_lo = t * kAT;  // the longest key tiles (most query tiles) first
  const long long hoff = static_cast<long long>(bh) * S * DK;
  const half_t* qg = static_cast<const half_t*>(a.q) + hoff;
  const half_t* og = static_cast<const half_t*>(a.dout) + static_cast<long long>(b) * S * a.H * DK + h * DK;
  constexpr int NB = 16 * DK / 8;
  stage16<DK>(Ks, nullptr, static_cast<const half_t*>(a.k) + hoff, DK, k_lo, S, 0);
  stage16<DK>(Vs, nullptr, static_cast<const half_t*>(a.v) + hoff, DK, k_lo, S, NB % 256);
  floatx16 dv[NJ], dk[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) dv[j][r] = dk[j][r] = 0.f;
  const int key = k_lo + 32 * wk + l32;
  const float inv_scale = 1.0f / a.scale, mul = score_mul<half_t>(a.scale);
  // At DK 64 each thread stages one block (threads 0-127 of Q, 128-255 of dO), so the next
  // query tile's block and statistics are fetched into registers while the current tile
  // is multiplied; at DK 128 (two blocks a thread) the registers are not there to spare.
  constexpr bool PF = NB == 128;
  const bool own_q = static_cast<int>(threadIdx.x) < NB;
  half8 nx[4];
  float nl = 0.f, nd = 0.f;
  auto fetch_next = [&](int lo) {
    if (own_q)
      fetch16<DK>(nx, qg, DK, lo, S, 0);
    else
      fetch16<DK>(nx, og, static_cast<long long>(a.H) * DK, lo, S, NB);
    if (threadIdx.x < kAT) {
      const int q = lo + threadIdx.x;
      nl = q < S ? a.lse[static_cast<long long>(bh) * S + q] : 0.f;
      nd = q < S ? a.dvec[static_cast<long long>(bh) * S + q] : 0.f;
    }
  };
  if constexpr (PF) fetch_next(k_lo);
  for (int q_lo = k_lo; q_lo < S; q_lo += kAT) {
    __syncthreads();
    if constexpr (PF) {
      if (own_q)
        put16<DK>(Qs, QT, nx, 0);
      else
        put16<DK>(Os, OT, nx, NB);
      if (threadIdx.x < kAT) {
        Ls[threadIdx.x] = nl;
        Ds[threadIdx.x] = nd;
      }
    } else {
      stage16<DK>(Qs, QT, qg, DK, q_lo, S, 0);
      stage16<DK>(Os, OT, og, static_cast<long long>(a.H) * DK, q_lo, S, NB % 256);
      if (threadIdx.x < kAT) {
        const int q = q_lo + threadIdx.x;
        Ls[threadIdx.x] = q < S ? a.lse[static_cast<long long>(bh) * S + q] : 0.f;
        Ds[threadIdx.x] = q < S ? a.dvec[static_cast<long long>(bh) * S + q] : 0.f;
      }
    }
    __syncthreads();
    if constexpr (PF)
      if (q_lo + kAT < S) fetch_next(q_lo + kAT);
    floatx16 sc, dp;
#pragma unroll
    for (int r = 0; r < 16; ++r) sc[r] = dp[r] = 0.f;
#pragma unroll
    for (int c0 = 0; c0 < DK; c0 += 16) {
      const half8 qa = *reinterpret_cast<const half8*>(Qs + (32 * wq + l32) * PA + c0 + 8 * hi);
      const half8 kb = *reinterpret_cast<const half8*>(Ks + (32 * wk + l32) * PA + c0 + 8 * hi);
      const half8 oa = *reinterpret_cast<const half8*>(Os + (32 * wq + l32) * PA + c0 + 8 * hi);
      const half8 vb = *reinterpret_cast<const half8*>(Vs + (32 * wk + l32) * PA + c0 + 8 * hi);
      sc = __builtin_amdgcn_mfma_f32_32x32x16_f16(qa, kb, sc, 0, 0, 0);
      dp = __builtin_amdgcn_mfma_f32_32x32x16_f16(oa, vb, dp, 0, 0, 0);
    }
    // The lane's 16 query rows are 32·wq + 8g + 4·hi + {0…3}, g < 4: their statistics as
    // four broadcast 16-byte reads each (not one conflicting scalar read a score), and
    // p = exp(s − lse) as exp2(s·log₂e − lse·log₂e). Only a tile that reaches past a
    // key's queries (the first) or past the sequence (the last) needs the mask.
    float nl2[16], dd[16];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const floatx4 l4 = *reinterpret_cast<const floatx4*>(Ls + 32 * wq + 8 * g + 4 * hi);
      const floatx4 d4 = *reinterpret_cast<const floatx4*>(Ds + 32 * wq + 8 * g + 4 * hi);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        nl2[4 * g + e] = -l4[e] * kLog2eF;
        dd[4 * g + e] = d4[e];
      }
    }
    if (q_lo < k_lo + kAT || q_lo + kAT > S) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int q = q_lo + 32 * wq + d_row(r, lane);
        float p = 0.f;
        if (key <= q && q < S)
          p = __builtin_amdgcn_exp2f(__builtin_fmaf(attn_score<half_t>(sc[r], mul), kLog2eF, nl2[r]));
        sc[r] = p;
        dp[r] = p * (dp[r] - dd[r]) * inv_scale;
      }
    } else {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(attn_score<half_t>(sc[r], mul), kLog2eF, nl2[r]));
        sc[r] = p;
        dp[r] = p * (dp[r] - dd[r]) * inv_scale;
      }
    }
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      const half8 pa = regs16(sc, st), sa = regs16(dp, st);
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        dv[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(pa, frag_t(OT, 32 * j, 32 * wq, st, lane), dv[j], 0, 0, 0);
        dk[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(sa, frag_t(QT, 32 * j, 32 * wq, st, lane), dk[j], 0, 0, 0);
      }
    }
  }
  __syncthreads();
  float* red = reinterpret_cast<float*>(Qs);  // 2 key halves × (dv, dk) × NJ × 16 × 64 floats
  if (wq == 1) {
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        red[(((wk * 2 + 0) * NJ + j) * 16 + r) * 64 + lane] = dv[j][r];
        red[(((wk * 2 + 1) * NJ + j) * 16 + r) * 64 + lane] = dk[j][r];
      }
  }
  __syncthreads();
  if (wq == 0) {
    const int d = a.H * DK;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int kk = k_lo + 32 * wk + d_row(r, lane);
      if (kk < S) {
        half_t* row = static_cast<half_t*>(a.dqkv) + (static_cast<long long>(b) * S + kk) * 3 * d + h * DK;
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
          row[d + 32 * j + l32] = static_cast<half_t>(dk[j][r] + red[(((wk * 2 + 1) * NJ + j) * 16 + r) * 64 + lane]);
          row[2 * d + 32 * j + l32] = static_cast<half_t>(dv[j][r] + red[(((wk * 2 + 0) * NJ + j) * 16 + r) * 64 + lane]);
        }
      }
    }
  }
}

template <int DK>
__global__ __launch_bounds__(256, 2) void attn_bwd_dq_f16(AttnBwdArgs a) {
  extern __shared__ __attribute__((aligned(16))) half_t lds16[];
  constexpr int PA = DK + 8, NJ = DK / 32, NB = 16 * DK / 8;
  half_t* Ks = lds16;
  half_t* Vs = Ks + kAT * PA;
  half_t* Qs = Vs + kAT * PA;
  half_t* Os = Qs + kAT * PA;
  half_t* KT = Os + kAT * PA;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, wk = w >> 1, wq = w & 1;
  const int l32 = lane & 31, hi = lane >> 5;
  int bh, t;
  bwd_tile_order(bh, t);
  const int b = bh / a.H, h = bh - (bh / a.H) * a.H;
  const int S = a.S, q_lo = (gridDim.x - 1 - t) * kAT;  // the longest query tiles first
  const long long hoff = static_cast<long long>(bh) * S * DK;
  const half_t* kg = static_cast<const half_t*>(a.k) + hoff;
  const half_t* vg = static_cast<const half_t*>(a.v) + hoff;
  stage16<DK>(Qs, nullptr, static_cast<const half_t*>(a.q) + hoff, DK, q_lo, S, 0);
  stage16<DK>(Os, nullptr,
              static_cast<const half_t*>(a.dout) + static_cast<long long>(b) * S * a.H * DK + h * DK,
              static_cast<long long>(a.H) * DK, q_lo, S, NB % 256);
  const int q = q_lo + 32 * wq + l32;
  const float lse = q < S ? a.lse[static_cast<long long>(bh) * S + q] : 0.f;
  const float dd = q < S ? a.dvec[static_cast<long long>(bh) * S + q] : 0.f;
  const float nlse2 = -lse * kLog2eF;
  const float inv_scale = 1.0f / a.scale, mul = score_mul<half_t>(a.scale);
  floatx16 dq[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) dq[j][r] = 0.f;
  const int k_end = min(S, q_lo + kAT);
  // DK 64: the next key tile's block (threads 0-127 of K, 128-255 of V) in registers while
  // the current one is multiplied, as in the dK/dV kernel
  constexpr bool PF = NB == 128;
  const bool own_k = static_cast<int>(threadIdx.x) < NB;
  half8 nx[4];
  auto fetch_next = [&](int lo) {
    if (own_k)
      fetch16<DK>(nx, kg, DK, lo, S, 0);
    else
      fetch16<DK>(nx, vg, DK, lo, S, NB);
  };
  if constexpr (PF) fetch_next(0);
  for (int k_lo = 0; k_lo < k_end; k_lo += kAT) {
    __syncthreads();
    if constexpr (PF) {
      if (own_k)
        put16<DK>(Ks, KT, nx, 0);
      else
        put16<DK>(Vs, nullptr, nx, NB);
    } else {
      stage16<DK>(Ks, KT, kg, DK, k_lo, S, 0);
      stage16<DK>(Vs, nullptr, vg, DK, k_lo, S, NB % 256);
    }
    __syncthreads();
    if constexpr (PF)
      if (k_lo + kAT < k_end) fetch_next(k_lo + kAT);
    floatx16 sc, dp;
#pragma unroll
    for (int r = 0; r < 16; ++r) sc[r] = dp[r] = 0.f;
#pragma unroll
    for (int c0 = 0; c0 < DK; c0 += 16) {
      const half8 ka = *reinterpret_cast<const half8*>(Ks + (32 * wk + l32) * PA + c0 + 8 * hi);
      const half8 qb = *reinterpret_cast<const half8*>(Qs + (32 * wq + l32) * PA + c0 + 8 * hi);
      const half8 va = *reinterpret_cast<const half8*>(Vs + (32 * wk + l32) * PA + c0 + 8 * hi);
      const half8 ob = *reinterpret_cast<const half8*>(Os + (32 * wq + l32) * PA + c0 + 8 * hi);
      sc = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka, qb, sc, 0, 0, 0);
      dp = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, ob, dp, 0, 0, 0);
    }
    // p = exp(s − lse) as exp2(s·log₂e − lse·log₂e); the mask only on the tile that
    // reaches past this workgroup's queries (the last) or a tile past the sequence
    if (k_lo + kAT > q_lo || q_lo + kAT > S) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int kk = k_lo + 32 * wk + d_row(r, lane);
        float p = 0.f;
        if (kk <= q && q < S)
          p = __builtin_amdgcn_exp2f(__builtin_fmaf(attn_score<half_t>(sc[r], mul), kLog2eF, nlse2));
        dp[r] = p * (dp[r] - dd) * inv_scale;
      }
    } else {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(attn_score<half_t>(sc[r], mul), kLog2eF, nlse2));
        dp[r] = p * (dp[r] - dd) * inv_scale;
      }
    }
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      const half8 sa = regs16(dp, st);
#pragma unroll
      for (int j = 0; j < NJ; ++j)
        dq[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(sa, frag_t(KT, 32 * j, 32 * wk, st, lane), dq[j], 0, 0, 0);
    }
  }
  __syncthreads();
  float* red = reinterpret_cast<float*>(lds16);  // 2 query halves × NJ × 16 × 64 floats
  if (wk == 1) {
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) red[((wq * NJ + j) * 16 + r) * 64 + lane] = dq[j][r];
  }
  __syncthreads();
  if (wk == 0) {
    const int d = a.H * DK;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int qq = q_lo + 32 * wq + d_row(r, lane);
      if (qq < S) {
        half_t* row = static_cast<half_t*>(a.dqkv) + (static_cast<long long>(b) * S + qq) * 3 * d + h * DK;
#pragma unroll
        for (int j = 0; j < NJ; ++j)
          row[32 * j + l32] = static_cast<half_t>(dq[j][r] + red[((wq * NJ + j) * 16 + r) * 64 + lane]);
      }
    }
  }
}

// The scalar pair (any head dim ≤ DK, tiles padded to DK columns).
template <int DK, typename T>
int attn_bwd_scalar(const AttnBwdArgs& a, hipStream_t st) {
  constexpr int BT = DK >= 128 ? 16 : 32;
  constexpr size_t lds = sizeof(AttnTile<DK, BT, T>);
  static bool attr = false;
  if (!attr) {
    NML_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(&attn_bwd_dkdv_kernel<DK, BT, T>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)));
    NML_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(&attn_bwd_dq_kernel<DK, BT, T>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)));
    attr = true;
  }
  const dim3 grid((a.S + BT - 1) / BT, a.B * a.H);
  attn_bwd_dkdv_kernel<DK, BT, T><<<grid, 256, lds, st>>>(a);
  NML_LAUNCHED();
  attn_bwd_dq_kernel<DK, BT, T><<<grid, 256, lds, st>>>(a);
  NML_LAUNCHED();
  return 0;
}

template <int DK>
int attn_bwd_f16(const AttnBwdArgs& a, hipStream_t st) {
  constexpr size_t lds = attn_f16_lds<DK>();
  static bool attr = false;
  if (!attr) {
    NML_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(&attn_bwd_dkdv_f16<DK>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)));
    NML_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(&attn_bwd_dq_f16<DK>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)));
    attr = true;
  }
  const dim3 grid((a.S + kAT - 1) / kAT, a.B * a.H);
  attn_bwd_dkdv_f16<DK><<<grid, 256, lds, st>>>(a);
  NML_LAUNCHED();
  attn_bwd_dq_f16<DK><<<grid, 256, lds, st>>>(a);
  NML_LAUNCHED();
  return 0;
}

template <int DK, typename T>
int attn_bwd_mfma(const AttnBwdArgs& a, hipStream_t st) {
  constexpr size_t lds = attn_mfma_lds<DK>();
  static bool attr = false;
  if (!attr) {
    NML_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(&attn_bwd_dkdv_mfma<DK, T>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)));
    NML_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(&attn_bwd_dq_mfma<DK, T>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)));
    attr = true;
  }
  const dim3 grid((a.S + kAT - 1) / kAT, a.B * a.H);
  attn_bwd_dkdv_mfma<DK, T><<<grid, 256, lds, st>>>(a);
  NML_LAUNCHED();
  attn_bwd_dq_mfma<DK, T><<<grid, 256, lds, st>>>(a);
  NML_LAUNCHED();
  return 0;
}

template <int DK, typename T>
int attn_bwd_dk(const AttnBwdArgs& a, hipStream_t st) {
  if constexpr (DK == 64 || DK == 128) {
    if (!a.full && !std::getenv("NIMBLEML_ATTN_BWD_VALU")) {  // MFMA kernels: causal only
      if constexpr (sizeof(T) == 2) {
        if (!std::getenv("NIMBLEML_TRAIN_F16_WIDEN")) return attn_bwd_f16<DK>(a, st);
      }
      return attn_bwd_mfma<DK, T>(a, st);
    }
  }
  return attn_bwd_scalar<DK, T>(a, st);
}

// --------------------------------------------------------------- RoPE backward
// The inverse rotation (utils/rope.py with inverse=True: sin negated), each product and
// sum in T (fp16 rounding points of apply_rope_flat).
template <typename T>
__global__ __launch_bounds__(256) void rope_bwd_kernel(T* __restrict__ dqkv, int rows, int S,
                                                       int H, int dk, const T* __restrict__ cs,
                                                       const T* __restrict__ sn) {
#pragma clang fp contract(off)
  const int half = dk / 2;
  const long long n = static_cast<long long>(rows) * 2 * H * half;
  const long long t = static_cast<long long>(blockIdx.x) * 256 + threadIdx.x;
  if (t >= n) return;
  const int i = static_cast<int>(t % half);
  const long long u = t / half;
  const int h = static_cast<int>(u % H);
  const int which = static_cast<int>((u / H) % 2);
  const int r = static_cast<int>(u / (2 * H));
  const int s = r % S;
  const int d = H * dk;
  T* p = dqkv + static_cast<long long>(r) * 3 * d + which * d + h * dk;
  const float c = static_cast<float>(cs[static_cast<long long>(s) * half + i]);
  const float si = static_cast<float>(sn[static_cast<long long>(s) * half + i]);
  const float x1 = static_cast<float>(p[i]), x2 = static_cast<float>(p[i + half]);
  p[i] = static_cast<T>(rnd<T>(x1 * c) + rnd<T>(x2 * si));
  p[i + half] = static_cast<T>(rnd<T>(x2 * c) - rnd<T>(x1 * si));
}

// ---------------------------------------------------------- embedding backward
template <typename T>
__global__ __launch_bounds__(256) void embed_bwd_tok_kernel(const T* __restrict__ g,
                                                            const int64_t* __restrict__ ids,
                                                            float* __restrict__ demb, int d, int V,
                                                            int n) {
  // demb[id] += the rows of g whose token is id, in ascending row order — the order of
  // the reference's scatter (kernels/embedding_scatter.py:39-80, np.add.at or the native
  // loop, called from layers/embedding.py:138-142) — so the sum does not
  // depend on scheduling. Block r does the work when row r is its id's first row: the
  // other blocks of that id find an earlier match and leave.
  const int r = blockIdx.x, t = threadIdx.x, w = t >> 6, lane = t & 63;
  const long long id = ids[r];
  if (id < 0 || id >= V) return;  // uniform over the block
  __shared__ int s_cnt[4];
  __shared__ int s_idx[256];
  for (int j0 = 0; j0 < r; j0 += 256) {
    const int j = j0 + t;
    if (__syncthreads_or(j < r && ids[j] == id)) return;
  }
  float* dst = demb + id * d;
  for (int j0 = r; j0 < n; j0 += 256) {
    const int j = j0 + t;
    const bool hit = j < n && ids[j] == id;
    const unsigned long long m = __ballot(hit);
    if (lane == 0) s_cnt[w] = __popcll(m);
    __syncthreads();
    int off = 0;
    for (int q = 0; q < w; ++q) off += s_cnt[q];
    const int tot = s_cnt[0] + s_cnt[1] + s_cnt[2] + s_cnt[3];
    if (hit) s_idx[off + __popcll(m & ((1ull << lane) - 1ull))] = j;
    __syncthreads();
    // each column read once, its rows added in ascending order in registers, stored
    // once: thread t owns 4 adjacent columns (one 8- or 16-byte load per row) and keeps 8
    // rows' loads in flight, so a frequent id (a pad token) costs a stream of loads rather
    // than a chain of read-modify-writes per row (d is a multiple of 4)
    for (int c = 4 * t; c < d; c += 1024) {
      float acc[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[e] = dst[c + e];
      for (int q0 = 0; q0 < tot; q0 += 8) {
        T v[8][4];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const int q = q0 + u < tot ? q0 + u : q0;  // past tot: a valid row, never added
          const T* src = g + static_cast<long long>(s_idx[q]) * d + c;
#pragma unroll
          for (int e = 0; e < 4; ++e) v[u][e] = src[e];
        }
#pragma unroll
        for (int u = 0; u < 8; ++u)
          if (q0 + u < tot)
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[e] += static_cast<float>(v[u][e]);
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) dst[c + e] = acc[e];
    }
    __syncthreads();
  }
}

template <typename T>
__global__ __launch_bounds__(256) void embed_bwd_pos_kernel(const T* __restrict__ g,
                                                            float* __restrict__ dpos, int B, int S,
                                                            int d) {
  const int s = blockIdx.y, c = blockIdx.x * 256 + threadIdx.x;
  if (c >= d) return;
  float v = 0.f;
  for (int b = 0; b < B; ++b) v += static_cast<float>(g[(static_cast<long long>(b) * S + s) * d + c]);
  dpos[static_cast<long long>(s) * d + c] += v;
}

template <typename S, typename D>
__global__ __launch_bounds__(256) void convert_kernel(const S* __restrict__ src, D* __restrict__ dst,
                                                      size_t n) {
  const size_t i = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i < n) dst[i] = static_cast<D>(static_cast<float>(src[i]));
}

}  // namespace

int launch_gemm_bwd(int dt, const GemmBwdArgs& g, bool a_kc, bool b_kc, int out, hipStream_t st) {
  if (g.M == 0 || g.N == 0) return 0;
  NML_REQUIRE(g.K > 0, "gemm_bwd: K must be positive");
  const uintptr_t al = dt == F16 ? 7 : 15;
  NML_REQUIRE(((reinterpret_cast<uintptr_t>(g.a) | reinterpret_cast<uintptr_t>(g.b)) & al) == 0 &&
                  g.lda % 4 == 0 && g.ldb % 4 == 0,
              "gemm_bwd: operands must be aligned to 4 elements with strides a multiple of 4");
  NML_REQUIRE(a_kc ? g.K % 4 == 0 : g.M % 4 == 0, "gemm_bwd: A's contiguous extent must be a multiple of 4");
  NML_REQUIRE(b_kc ? g.K % 4 == 0 : g.N % 4 == 0, "gemm_bwd: B's contiguous extent must be a multiple of 4");
  NML_REQUIRE(out != GB_GELU || g.aux != nullptr, "gemm_bwd: the GELU backward needs the pre-activation");
  if (dt == F16) {
    // 16-byte fp16 pieces: the contiguous extent of each operand a multiple of 8 elements
    const bool m16 = !std::getenv("NIMBLEML_TRAIN_F16_WIDEN") &&
                     ((reinterpret_cast<uintptr_t>(g.a) | reinterpret_cast<uintptr_t>(g.b)) & 15) == 0 &&
                     g.lda % 8 == 0 && g.ldb % 8 == 0 && (a_kc ? g.K % 8 == 0 : g.M % 8 == 0) &&
                     (b_kc ? g.K % 8 == 0 : g.N % 8 == 0);
    const char* bigenv = std::getenv("NIMBLEML_TRAIN_F16_BIG");
    if (m16 && g.K % big::kK == 0 && !(bigenv && bigenv[0] == '0')) return gemm_bwd_big(g, a_kc, b_kc, out, st);
    if (a_kc)
      return b_kc ? gemm_bwd_out<true, true, half_t>(g, out, st, m16) : gemm_bwd_out<true, false, half_t>(g, out, st, m16);
    return b_kc ? gemm_bwd_out<false, true, half_t>(g, out, st, m16) : gemm_bwd_out<false, false, half_t>(g, out, st, m16);
  }
  if (a_kc) return b_kc ? gemm_bwd_out<true, true, float>(g, out, st) : gemm_bwd_out<true, false, float>(g, out, st);
  return b_kc ? gemm_bwd_out<false, true, float>(g, out, st) : gemm_bwd_out<false, false, float>(g, out, st);
}

int launch_convert(int src_dt, const void* src, int dst_dt, void* dst, size_t n, hipStream_t st) {
  if (n == 0) return 0;
  const size_t blocks = (n + 255) / 256;
  NML_REQUIRE(blocks <= 0x7fffffff, "convert: %zu elements exceed one launch", n);
  if (src_dt == F16 && dst_dt == F32)
    convert_kernel<half_t, float><<<static_cast<int>(blocks), 256, 0, st>>>(
        static_cast<const half_t*>(src), static_cast<float*>(dst), n);
  else if (src_dt == F32 && dst_dt == F16)
    convert_kernel<float, half_t><<<static_cast<int>(blocks), 256, 0, st>>>(
        static_cast<const float*>(src), static_cast<half_t*>(dst), n);
  else {
    set_error("convert: unsupported dtypes %d -> %d", src_dt, dst_dt);
    return -1;
  }
  NML_LAUNCHED();
  return 0;
}

int rmsnorm_bwd_parts(int rows) { return (rows + kNormRowsPerWave - 1) / kNormRowsPerWave; }

int launch_rmsnorm_bwd(int dt, const void* dy, const void* x, const void* gamma, void* dx, int acc,
                       float* dgamma, float* part, int rows, int d, float eps, hipStream_t st) {
  if (rows == 0) return 0;
  const int waves = (rows + kNormRowsPerWave - 1) / kNormRowsPerWave;
  const int blocks = (rows + kNormRowsPerBlock - 1) / kNormRowsPerBlock;
  const int nv = (d / 4 + 63) / 64;
  const uintptr_t al = dt == F16 ? 7 : 15;
  const bool vec_ok = d % 4 == 0 && ((reinterpret_cast<uintptr_t>(dy) | reinterpret_cast<uintptr_t>(x) |
                                      reinterpret_cast<uintptr_t>(gamma) |
                                      reinterpret_cast<uintptr_t>(dx)) & al) == 0;
  if (vec_ok && nv <= 8) {
    const int wblocks = (waves + 3) / 4;
#define NML_NORM_BWD_W(T, NVV)                                                                   \
  rmsnorm_bwd_wave_kernel<T, NVV><<<wblocks, 256, 0, st>>>((const T*)dy, (const T*)x, (const T*)gamma, \
                                                          (T*)dx, acc, part, rows, d, eps)
    if (dt == F16) {
      if (nv <= 1) NML_NORM_BWD_W(half_t, 1);
      else if (nv <= 2) NML_NORM_BWD_W(half_t, 2);
      else if (nv <= 4) NML_NORM_BWD_W(half_t, 4);
      else NML_NORM_BWD_W(half_t, 8);
    } else {
      if (nv <= 1) NML_NORM_BWD_W(float, 1);
      else if (nv <= 2) NML_NORM_BWD_W(float, 2);
      else if (nv <= 4) NML_NORM_BWD_W(float, 4);
      else NML_NORM_BWD_W(float, 8);
    }
#undef NML_NORM_BWD_W
    NML_LAUNCHED();
    parts_reduce_kernel<<<(d + 31) / 32, 256, 0, st>>>(part, wblocks, d, dgamma);
    NML_LAUNCHED();
    return 0;
  }
  NML_REQUIRE(dt == F32, "rmsnorm backward: fp16 needs d %% 4 == 0, d <= 2048 and aligned rows");
  NML_REQUIRE(d > 0 && d <= 256 * 32, "rmsnorm backward: d=%d outside (0, 8192]", d);
  const int nc = (d + 255) / 256;
  const float* fdy = static_cast<const float*>(dy);
  const float* fx = static_cast<const float*>(x);
  const float* fg = static_cast<const float*>(gamma);
  float* fdx = static_cast<float*>(dx);
#define NML_NORM_BWD(NCV) \
  rmsnorm_bwd_kernel<NCV><<<blocks, 256, 0, st>>>(fdy, fx, fg, fdx, acc, part, rows, d, eps)
  if (nc <= 1) NML_NORM_BWD(1);
  else if (nc <= 2) NML_NORM_BWD(2);
  else if (nc <= 4) NML_NORM_BWD(4);
  else if (nc <= 8) NML_NORM_BWD(8);
  else if (nc <= 16) NML_NORM_BWD(16);
  else NML_NORM_BWD(32);
#undef NML_NORM_BWD
  NML_LAUNCHED();
  parts_reduce_kernel<<<(d + 31) / 32, 256, 0, st>>>(part, blocks, d, dgamma);
  NML_LAUNCHED();
  return 0;
}

int colsum_parts(int rows) { return (rows + kColRows - 1) / kColRows; }

int launch_colsum(int dt, const void* a, long long lda, int rows, int n, float* out, float* part,
                  hipStream_t st) {
  if (rows == 0 || n == 0) return 0;
  const int parts = colsum_parts(rows);
  const int vec = dt == F16 ? 8 : 4;
  const bool wide = n % vec == 0 && lda % vec == 0 && (reinterpret_cast<uintptr_t>(a) & 15) == 0;
  const int span = 32 * (wide ? vec : 1);
  const dim3 grid((n + span - 1) / span, parts);
  if (dt == F16) {
    const half_t* h = static_cast<const half_t*>(a);
    if (wide)
      colsum_part_kernel<half_t, 8><<<grid, 256, 0, st>>>(h, lda, rows, n, part);
    else
      colsum_part_kernel<half_t, 1><<<grid, 256, 0, st>>>(h, lda, rows, n, part);
  } else {
    const float* f = static_cast<const float*>(a);
    if (wide)
      colsum_part_kernel<float, 4><<<grid, 256, 0, st>>>(f, lda, rows, n, part);
    else
      colsum_part_kernel<float, 1><<<grid, 256, 0, st>>>(f, lda, rows, n, part);
  }
  NML_LAUNCHED();
  parts_reduce_kernel<<<(n + 31) / 32, 256, 0, st>>>(part, parts, n, out);
  NML_LAUNCHED();
  return 0;
}

int launch_ce_grad(int dt, void* logits, int rows, int V, const int64_t* labels,
                   long long ignore_index, int has_ignore, float scale, hipStream_t st) {
  if (rows == 0) return 0;
  // rows in registers when the row is whole 16-byte chunks, ≤ 8192 of them, and aligned
  const int E = dt == F16 ? 8 : 4;
  const int nch = V / E, per = (nch + 255) / 256;
  if (V % E == 0 && per <= 32 && (reinterpret_cast<uintptr_t>(logits) & 15) == 0) {
    if (dt == F16) {
      half_t* l = static_cast<half_t*>(logits);
      if (per <= 4) ce_grad_reg_kernel<half_t, 4><<<rows, 256, 0, st>>>(l, V, labels, ignore_index, has_ignore, scale);
      else if (per <= 16) ce_grad_reg_kernel<half_t, 16><<<rows, 256, 0, st>>>(l, V, labels, ignore_index, has_ignore, scale);
      else ce_grad_reg_kernel<half_t, 32><<<rows, 256, 0, st>>>(l, V, labels, ignore_index, has_ignore, scale);
    } else {
      float* l = static_cast<float*>(logits);
      if (per <= 4) ce_grad_reg_kernel<float, 4><<<rows, 256, 0, st>>>(l, V, labels, ignore_index, has_ignore, scale);
      else if (per <= 16) ce_grad_reg_kernel<float, 16><<<rows, 256, 0, st>>>(l, V, labels, ignore_index, has_ignore, scale);
      else ce_grad_reg_kernel<float, 32><<<rows, 256, 0, st>>>(l, V, labels, ignore_index, has_ignore, scale);
    }
    NML_LAUNCHED();
    return 0;
  }
  if (dt == F16)
    ce_grad_kernel<half_t><<<rows, 256, 0, st>>>(static_cast<half_t*>(logits), V, labels, ignore_index,
                                                 has_ignore, scale);
  else
    ce_grad_kernel<float><<<rows, 256, 0, st>>>(static_cast<float*>(logits), V, labels, ignore_index,
                                                has_ignore, scale);
  NML_LAUNCHED();
  return 0;
}

template <typename T>
int attention_backward_t(const AttnBwdArgs& a, hipStream_t st) {
  const long long pairs = static_cast<long long>(a.B) * a.S * a.H;
  attn_bwd_dot_kernel<T><<<static_cast<int>((pairs + 3) / 4), 256, 0, st>>>(a);
  NML_LAUNCHED();
  switch (a.dk) {
    case 8: return attn_bwd_dk<8, T>(a, st);
    case 16: return attn_bwd_dk<16, T>(a, st);
    case 32: return attn_bwd_dk<32, T>(a, st);
    case 64: return attn_bwd_dk<64, T>(a, st);
    case 128: return attn_bwd_dk<128, T>(a, st);
  }
  // other head dims: the scalar kernels on tiles padded to 32, 64, 128 or 256 columns
  if (a.dk < 1 || a.dk > kMaxHeadDim) {
    set_error("attention backward: head_dim %d outside [1, %d]", a.dk, kMaxHeadDim);
    return -1;
  }
  if (a.dk <= 32) return attn_bwd_scalar<32, T>(a, st);
  if (a.dk <= 64) return attn_bwd_scalar<64, T>(a, st);
  if (a.dk <= 128) return attn_bwd_scalar<128, T>(a, st);
  return attn_bwd_scalar<256, T>(a, st);
}

int launch_attention_backward(int dt, const AttnBwdArgs& a, hipStream_t st) {
  if (a.B * a.S == 0) return 0;
  NML_REQUIRE(a.full || !a.mask, "attention backward: a causal call takes no mask");
  return dt == F16 ? attention_backward_t<half_t>(a, st) : attention_backward_t<float>(a, st);
}

int launch_rope_backward(int dt, void* dqkv, int rows, int S, int H, int dk, const void* cos,
                         const void* sin, hipStream_t st) {
  const long long n = static_cast<long long>(rows) * 2 * H * (dk / 2);
  if (n == 0) return 0;
  const int blocks = static_cast<int>((n + 255) / 256);
  if (dt == F16)
    rope_bwd_kernel<half_t><<<blocks, 256, 0, st>>>(static_cast<half_t*>(dqkv), rows, S, H, dk,
                                                    static_cast<const half_t*>(cos),
                                                    static_cast<const half_t*>(sin));
  else
    rope_bwd_kernel<float><<<blocks, 256, 0, st>>>(static_cast<float*>(dqkv), rows, S, H, dk,
                                                   static_cast<const float*>(cos),
                                                   static_cast<const float*>(sin));
  NML_LAUNCHED();
  return 0;
}

int launch_embed_backward(int dt, const void* g, const int64_t* ids, float* demb, float* dpos, int B,
                          int S, int d, int V, hipStream_t st) {
  if (B * S == 0) return 0;
  if (dt == F16)
    embed_bwd_tok_kernel<half_t><<<B * S, 256, 0, st>>>(static_cast<const half_t*>(g), ids, demb, d, V, B * S);
  else
    embed_bwd_tok_kernel<float><<<B * S, 256, 0, st>>>(static_cast<const float*>(g), ids, demb, d, V, B * S);
  NML_LAUNCHED();
  if (dpos) {
    const dim3 grid((d + 255) / 256, S);
    if (dt == F16)
      embed_bwd_pos_kernel<half_t><<<grid, 256, 0, st>>>(static_cast<const half_t*>(g), dpos, B, S, d);
    else
      embed_bwd_pos_kernel<float><<<grid, 256, 0, st>>>(static_cast<const float*>(g), dpos, B, S, d);
    NML_LAUNCHED();
  }
  return 0;
}

}  // namespace nml
