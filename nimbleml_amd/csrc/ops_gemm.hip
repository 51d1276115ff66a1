// Projections out = epi(x · Wᵀ): QKV, W_o, W1, W2 and the tied LM head.
//
// Weights live on device transposed to (out, in) = (N, K), K-contiguous, so both
// GEMM operands are K-major (the natural MFMA operand layout) and a decode GEMV
// streams each output's weights as one contiguous row.
//
//  * gemm_f16 / gemm_f32: 128×128 block tile, 4 waves as 2×2, each wave 64×64 as
//    2×2 MFMA 32×32 tiles (fp16: v_mfma_f32_32x32x16_f16, K=64 per LDS stage;
//    fp32: v_mfma_f32_32x32x2f32, K=32 per stage). Next stage prefetched into
//    registers while the current one is multiplied.
//  * gemv: M ≤ 8 activation rows (decode). One wave per output row (or four),
//    16-byte loads along K, fp32 accumulation, wave-reduced.
#include "kernels.hpp"

namespace nml {

namespace {

template <typename T, int EPI>
__device__ __forceinline__ void epilogue(const LinearArgs& a, int m, int n, float acc) {
  T* out = static_cast<T*>(a.out);
  const size_t idx = static_cast<size_t>(m) * a.N + n;
  if constexpr (EPI == EPI_NONE) {
    out[idx] = static_cast<T>(acc);
  } else {
    const float lin = rnd<T>(rnd<T>(acc) + static_cast<float>(static_cast<const T*>(a.bias)[n]));
    if constexpr (EPI == EPI_BIAS) {
      out[idx] = static_cast<T>(lin);
    } else if constexpr (EPI == EPI_BIAS_GELU) {
      out[idx] = static_cast<T>(gelu_t<T>(lin));
    } else if constexpr (EPI == EPI_BIAS_RESID) {
      out[idx] = static_cast<T>(static_cast<float>(static_cast<const T*>(a.resid)[idx]) + lin);
    } else {  // EPI_QKV
      const QKVDst& q = a.qkv;
      const int which = n / q.d;
      const int within = n - which * q.d;
      const int h = within / q.dk, j = within - h * q.dk;
      const int b = m / q.S, s = m - b * q.S;
      if (which == 0) {
        T* qp = static_cast<T*>(q.q);
        qp[((static_cast<size_t>(b) * q.H + h) * q.S + s) * q.dk + j] = static_cast<T>(lin);
      } else {
        const int pos = (q.pos_base ? q.pos_base[b] : 0) + s;
        T* kv = static_cast<T*>(which == 1 ? q.k : q.v);
        kv[b * q.kv_stride_b + h * q.kv_stride_h + static_cast<long long>(pos) * q.dk + j] =
            static_cast<T>(lin);
      }
    }
  }
}

constexpr int kBM = 128, kBN = 128;

// ---------------------------------------------------------------- fp16 MFMA GEMM
constexpr int kBK16 = 64, kPad16 = 8;

template <int EPI>
__global__ __launch_bounds__(256) void gemm_f16_kernel(LinearArgs a) {
  __shared__ half_t As[kBM][kBK16 + kPad16];
  __shared__ half_t Bs[kBN][kBK16 + kPad16];
  const half_t* __restrict__ X = static_cast<const half_t*>(a.x);
  const half_t* __restrict__ W = static_cast<const half_t*>(a.w);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int m0 = blockIdx.y * kBM, n0 = blockIdx.x * kBN;
  const int M = a.M, N = a.N, K = a.K;
  const long long lda = a.lda;

  floatx16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  half8 ra[4], rb[4];
  const half8 zero8 = {0, 0, 0, 0, 0, 0, 0, 0};
  auto gload = [&](int k0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = tid + 256 * i;
      const int row = c >> 3, kc = (c & 7) * 8;
      const int gk = k0 + kc;
      const int gm = m0 + row, gn = n0 + row;
      ra[i] = (gm < M && gk < K) ? *reinterpret_cast<const half8*>(X + gm * lda + gk) : zero8;
      rb[i] = (gn < N && gk < K)
                  ? *reinterpret_cast<const half8*>(W + static_cast<long long>(gn) * K + gk)
                  : zero8;
    }
  };
  auto sstore = [&]() {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = tid + 256 * i;
      const int row = c >> 3, kc = (c & 7) * 8;
      *reinterpret_cast<half8*>(&As[row][kc]) = ra[i];
      *reinterpret_cast<half8*>(&Bs[row][kc]) = rb[i];
    }
  };

  gload(0);
  sstore();
  __syncthreads();
  for (int k0 = 0; k0 < K; k0 += kBK16) {
    const bool more = k0 + kBK16 < K;
    if (more) gload(k0 + kBK16);
#pragma unroll
    for (int kk = 0; kk < kBK16; kk += 16) {
      half8 fa[2], fb[2];
#pragma unroll
      for (int i = 0; i < 2; ++i)
        fa[i] = *reinterpret_cast<const half8*>(&As[wm * 64 + i * 32 + (lane & 31)][kk + (lane >> 5) * 8]);
#pragma unroll
      for (int j = 0; j < 2; ++j)
        fb[j] = *reinterpret_cast<const half8*>(&Bs[wn * 64 + j * 32 + (lane & 31)][kk + (lane >> 5) * 8]);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa[i], fb[j], acc[i][j], 0, 0, 0);
    }
    __syncthreads();
    if (more) sstore();
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
        if (m < M && n < N) epilogue<half_t, EPI>(a, m, n, acc[i][j][r]);
      }
}

// ---------------------------------------------------------------- fp32 MFMA GEMM
constexpr int kBK32 = 32, kPad32 = 4;

template <int EPI>
__global__ __launch_bounds__(256) void gemm_f32_kernel(LinearArgs a) {
  __shared__ float As[kBM][kBK32 + kPad32];
  __shared__ float Bs[kBN][kBK32 + kPad32];
  const float* __restrict__ X = static_cast<const float*>(a.x);
  const float* __restrict__ W = static_cast<const float*>(a.w);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int m0 = blockIdx.y * kBM, n0 = blockIdx.x * kBN;
  const int M = a.M, N = a.N, K = a.K;
  const long long lda = a.lda;

  floatx16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  floatx4 ra[4], rb[4];
  const floatx4 zero4 = {0.f, 0.f, 0.f, 0.f};
  auto gload = [&](int k0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = tid + 256 * i;
      const int row = c >> 3, kc = (c & 7) * 4;
      const int gk = k0 + kc;
      const int gm = m0 + row, gn = n0 + row;
      ra[i] = (gm < M && gk < K) ? *reinterpret_cast<const floatx4*>(X + gm * lda + gk) : zero4;
      rb[i] = (gn < N && gk < K)
                  ? *reinterpret_cast<const floatx4*>(W + static_cast<long long>(gn) * K + gk)
                  : zero4;
    }
  };
  auto sstore = [&]() {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = tid + 256 * i;
      const int row = c >> 3, kc = (c & 7) * 4;
      *reinterpret_cast<floatx4*>(&As[row][kc]) = ra[i];
      *reinterpret_cast<floatx4*>(&Bs[row][kc]) = rb[i];
    }
  };

  gload(0);
  sstore();
  __syncthreads();
  for (int k0 = 0; k0 < K; k0 += kBK32) {
    const bool more = k0 + kBK32 < K;
    if (more) gload(k0 + kBK32);
#pragma unroll
    for (int kk = 0; kk < kBK32; kk += 2) {
      float fa[2], fb[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) fa[i] = As[wm * 64 + i * 32 + (lane & 31)][kk + (lane >> 5)];
#pragma unroll
      for (int j = 0; j < 2; ++j) fb[j] = Bs[wn * 64 + j * 32 + (lane & 31)][kk + (lane >> 5)];
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[i], fb[j], acc[i][j], 0, 0, 0);
    }
    __syncthreads();
    if (more) sstore();
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
        if (m < M && n < N) epilogue<float, EPI>(a, m, n, acc[i][j][r]);
      }
}

// --------------------------------------------------------------------- GEMV
template <typename T>
struct Vec16;
template <>
struct Vec16<half_t> {
  typedef half8 type;
  static constexpr int n = 8;
};
template <>
struct Vec16<float> {
  typedef floatx4 type;
  static constexpr int n = 4;
};

template <typename T, int EPI, int MR, int RPW>
__global__ __launch_bounds__(256) void gemv_kernel(LinearArgs a) {
  using V = typename Vec16<T>::type;
  constexpr int VN = Vec16<T>::n;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nbase = (blockIdx.x * 4 + wave) * RPW;
  const T* __restrict__ X = static_cast<const T*>(a.x);
  const T* __restrict__ W = static_cast<const T*>(a.w);
  const int M = a.M, N = a.N, K = a.K;
  float acc[RPW][MR];
#pragma unroll
  for (int r = 0; r < RPW; ++r)
#pragma unroll
    for (int m = 0; m < MR; ++m) acc[r][m] = 0.f;

  for (int k = lane * VN; k < K; k += 64 * VN) {
    V w[RPW];
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
      const int n = nbase + r;
      if (n < N) {
        w[r] = *reinterpret_cast<const V*>(W + static_cast<long long>(n) * K + k);
      } else {
#pragma unroll
        for (int e = 0; e < VN; ++e) w[r][e] = static_cast<T>(0.f);
      }
    }
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      if (m < M) {
        const V xv = *reinterpret_cast<const V*>(X + m * a.lda + k);
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
          float s = 0.f;
#pragma unroll
          for (int e = 0; e < VN; ++e) s += static_cast<float>(w[r][e]) * static_cast<float>(xv[e]);
          acc[r][m] += s;
        }
      }
    }
  }
#pragma unroll
  for (int r = 0; r < RPW; ++r)
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      const float s = wave_sum(acc[r][m]);
      const int n = nbase + r;
      if (lane == 0 && m < M && n < N) epilogue<T, EPI>(a, m, n, s);
    }
}

template <typename T, int EPI, int MR>
int gemv_dispatch_rpw(const LinearArgs& a, hipStream_t st) {
  if (a.N >= 8192) {
    const int blocks = (a.N + 15) / 16;
    gemv_kernel<T, EPI, MR, 4><<<blocks, 256, 0, st>>>(a);
  } else {
    const int blocks = (a.N + 3) / 4;
    gemv_kernel<T, EPI, MR, 1><<<blocks, 256, 0, st>>>(a);
  }
  NML_LAUNCHED();
  return 0;
}

template <typename T, int EPI>
int linear_typed(const LinearArgs& a, hipStream_t st) {
  if (a.M <= 8) {
    if (a.M <= 1) return gemv_dispatch_rpw<T, EPI, 1>(a, st);
    if (a.M <= 2) return gemv_dispatch_rpw<T, EPI, 2>(a, st);
    if (a.M <= 4) return gemv_dispatch_rpw<T, EPI, 4>(a, st);
    return gemv_dispatch_rpw<T, EPI, 8>(a, st);
  }
  dim3 grid((a.N + kBN - 1) / kBN, (a.M + kBM - 1) / kBM);
  if constexpr (sizeof(T) == 2)
    gemm_f16_kernel<EPI><<<grid, 256, 0, st>>>(a);
  else
    gemm_f32_kernel<EPI><<<grid, 256, 0, st>>>(a);
  NML_LAUNCHED();
  return 0;
}

template <typename T>
int linear_epi(const LinearArgs& a, hipStream_t st) {
  switch (a.epi) {
    case EPI_NONE: return linear_typed<T, EPI_NONE>(a, st);
    case EPI_BIAS: return linear_typed<T, EPI_BIAS>(a, st);
    case EPI_BIAS_GELU: return linear_typed<T, EPI_BIAS_GELU>(a, st);
    case EPI_BIAS_RESID: return linear_typed<T, EPI_BIAS_RESID>(a, st);
    case EPI_QKV: return linear_typed<T, EPI_QKV>(a, st);
  }
  set_error("unknown epilogue %d", a.epi);
  return -1;
}

}  // namespace

int launch_linear(int dt, const LinearArgs& a, hipStream_t st) {
  if (a.M == 0 || a.N == 0) return 0;
  const int vec = dt == F16 ? 8 : 4;
  NML_REQUIRE(a.K > 0 && a.K % vec == 0, "linear: K=%d must be a positive multiple of %d", a.K, vec);
  NML_REQUIRE(a.lda % vec == 0, "linear: row stride %lld must be a multiple of %d", a.lda, vec);
  NML_REQUIRE((reinterpret_cast<uintptr_t>(a.x) & 15) == 0 &&
                  (reinterpret_cast<uintptr_t>(a.w) & 15) == 0,
              "linear: x and w must be 16-byte aligned");
  NML_REQUIRE(a.epi == EPI_NONE || a.bias != nullptr, "linear: epilogue %d needs a bias", a.epi);
  NML_REQUIRE(a.epi != EPI_BIAS_RESID || a.resid != nullptr, "linear: residual pointer missing");
  NML_REQUIRE(a.epi != EPI_QKV || (a.qkv.d > 0 && a.qkv.dk > 0 && a.N == 3 * a.qkv.d &&
                                   a.M == a.qkv.S * (a.M / a.qkv.S)),
              "linear: bad QKV destination");
  return dt == F16 ? linear_epi<half_t>(a, st) : linear_epi<float>(a, st);
}

}  // namespace nml
