// Row-wise and elementwise kernels: embedding gather + position add, RMSNorm,
// tanh-GELU. All are HBM-bound; one workgroup (256 lanes, 4 waves) per row.
#include "kernels.hpp"

namespace nml {

namespace {

// x = E[ids] + P[pos]  (models/gpt.py:85-86; gather kernels/embedding_scatter.py:25-36,
// position prefix layers/embedding.py:72-118). fp16 + fp16 computed in fp32 and rounded
// once is the correctly rounded fp16 sum, i.e. NumPy's fp16 add: bit-exact. With rotary
// positions there is no P (posw null, models/gpt.py:85): x = E[ids].
template <typename T>
__global__ __launch_bounds__(256) void embed_kernel(const int64_t* __restrict__ ids,
                                                    const T* __restrict__ emb,
                                                    const T* __restrict__ posw,
                                                    const int32_t* __restrict__ pos_base,
                                                    T* __restrict__ out, int S, int d, int V,
                                                    int P, int* __restrict__ err) {
  const int row = blockIdx.x;
  const int b = row / S, s = row - b * S;
  const int64_t id = ids[row];
  const int p = (pos_base ? pos_base[b] : 0) + s;
  T* o = out + static_cast<size_t>(row) * d;
  if (id < 0 || id >= V || p < 0 || p >= P) {
    if (threadIdx.x == 0 && err) atomicOr(err, 1);
    for (int j = threadIdx.x; j < d; j += blockDim.x) o[j] = static_cast<T>(0.f);
    return;
  }
  const T* e = emb + static_cast<size_t>(id) * d;
  if (!posw) {
    for (int j = threadIdx.x; j < d; j += blockDim.x) o[j] = e[j];
    return;
  }
  const T* q = posw + static_cast<size_t>(p) * d;
  for (int j = threadIdx.x; j < d; j += blockDim.x)
    o[j] = static_cast<T>(static_cast<float>(e[j]) + static_cast<float>(q[j]));
}

template <typename T>
__global__ __launch_bounds__(256) void embed_decode_kernel(
    const int64_t* __restrict__ tokens, long long tok_stride, const int32_t* __restrict__ pos,
    const T* __restrict__ emb, const T* __restrict__ posw, T* __restrict__ out, int d, int V,
    int P, int* __restrict__ err) {
  const int b = blockIdx.x;
  const int p = pos[b];
  const int64_t id = (p >= 0) ? tokens[b * tok_stride + p] : -1;
  T* o = out + static_cast<size_t>(b) * d;
  if (id < 0 || id >= V || p < 0 || p >= P) {
    if (threadIdx.x == 0 && err) atomicOr(err, 1);
    for (int j = threadIdx.x; j < d; j += blockDim.x) o[j] = static_cast<T>(0.f);
    return;
  }
  const T* e = emb + static_cast<size_t>(id) * d;
  if (!posw) {
    for (int j = threadIdx.x; j < d; j += blockDim.x) o[j] = e[j];
    return;
  }
  const T* q = posw + static_cast<size_t>(p) * d;
  for (int j = threadIdx.x; j < d; j += blockDim.x)
    o[j] = static_cast<T>(static_cast<float>(e[j]) + static_cast<float>(q[j]));
}

// Rotary positions, GPT-NeoX half split (utils/rope.py:22-44): dims (i, i + dk/2) of a
// row at position p become (x1·c − x2·s, x1·s + x2·c) with c = cos[p][i], s = sin[p][i]
// in the compute dtype; each product and the sum/difference is one op of the storage
// type (fp16: float32 result rounded once to fp16, NumPy's fp16 op; no contraction).
// One thread per (row, pair); q and the cached K row are rotated in place.
template <typename T>
__global__ __launch_bounds__(256) void rope_kernel(T* __restrict__ q, T* __restrict__ k,
                                                   long long sb, long long sh, int H, int S,
                                                   int dk, const int32_t* __restrict__ pos_base,
                                                   const int32_t* __restrict__ seq_len,
                                                   const T* __restrict__ cosv,
                                                   const T* __restrict__ sinv, int max_len) {
#pragma clang fp contract(off)
  const int half = dk / 2;
  const int bh = blockIdx.y, b = bh / H, h = bh - b * H;
  const int idx = blockIdx.x * blockDim.x + threadIdx.x;  // row · half + pair
  const int s = idx / half, i = idx - s * half;
  if (s >= S || (seq_len && s >= seq_len[b])) return;
  const int p = (pos_base ? pos_base[b] : 0) + s;
  if (p < 0 || p >= max_len) return;
  const float c = static_cast<float>(cosv[static_cast<size_t>(p) * half + i]);
  const float sn = static_cast<float>(sinv[static_cast<size_t>(p) * half + i]);
  auto rot = [&](T* row) {
    const float x1 = static_cast<float>(row[i]), x2 = static_cast<float>(row[i + half]);
    const float a = rnd<T>(rnd<T>(x1 * c) - rnd<T>(x2 * sn));
    const float bb = rnd<T>(rnd<T>(x1 * sn) + rnd<T>(x2 * c));
    row[i] = static_cast<T>(a);
    row[i + half] = static_cast<T>(bb);
  };
  rot(q + (static_cast<size_t>(bh) * S + s) * dk);
  rot(k + b * sb + h * sh + static_cast<long long>(p) * dk);
}

// RMSNorm (kernels/fused_rmsnorm.py:153-162).
//   fp32: ms = mean(x²); rms = sqrt(ms + eps); y = (x / rms) · γ
//   fp16: x² rounded to fp16, mean accumulated in fp32; inv = fp16(1 / rms);
//         y = fp16(fp16(x · inv) · γ)
template <typename T>
__global__ __launch_bounds__(256) void rmsnorm_kernel(const T* __restrict__ x,
                                                      const T* __restrict__ g,
                                                      T* __restrict__ out, float* __restrict__ ms,
                                                      float* __restrict__ rmsv, int d, float eps) {
#pragma clang fp contract(off)
  __shared__ float red[16];
  const int row = blockIdx.x;
  const T* xr = x + static_cast<size_t>(row) * d;
  T* o = out + static_cast<size_t>(row) * d;
  float acc = 0.f;
  for (int j = threadIdx.x; j < d; j += blockDim.x) {
    const float v = static_cast<float>(xr[j]);
    acc += rnd<T>(v * v);
  }
  const float m = block_sum(acc, red) / static_cast<float>(d);
  const float r = sqrtf(m + eps);
  if (threadIdx.x == 0) {
    if (ms) ms[row] = m;
    if (rmsv) rmsv[row] = r;
  }
  if constexpr (sizeof(T) == 2) {
    const float inv = rnd<T>(1.0f / r);
    for (int j = threadIdx.x; j < d; j += blockDim.x) {
      const float v = rnd<T>(static_cast<float>(xr[j]) * inv);
      o[j] = static_cast<T>(v * static_cast<float>(g[j]));
    }
  } else {
    for (int j = threadIdx.x; j < d; j += blockDim.x)
      o[j] = static_cast<T>((static_cast<float>(xr[j]) / r) * static_cast<float>(g[j]));
  }
}

// The same RMSNorm with one wave per row (4 rows per workgroup): each lane keeps its NV
// 16-byte vectors of the row in registers between the sum of squares (DPP wave sum, no
// LDS, no barrier) and the scaling, so the row is read once. Requires d ≤ NV·64 vectors.
template <typename T, int NV>
__global__ __launch_bounds__(256) void rmsnorm_wave_kernel(const T* __restrict__ x,
                                                           const T* __restrict__ g,
                                                           T* __restrict__ out, float* __restrict__ ms,
                                                           float* __restrict__ rmsv, int rows, int d,
                                                           float eps) {
#pragma clang fp contract(off)
  typedef float vf __attribute__((ext_vector_type(4)));
  constexpr int E = 16 / sizeof(T);  // elements per vector
  typedef T vec __attribute__((ext_vector_type(E)));
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;  // whole waves
  const int nvec = d / E;
  const vec* xr = reinterpret_cast<const vec*>(x + static_cast<size_t>(row) * d);
  vec xv[NV];
  float acc = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int c = lane + 64 * i;
    if (c < nvec) {
      xv[i] = xr[c];
#pragma unroll
      for (int e = 0; e < E; ++e) {
        const float v = static_cast<float>(xv[i][e]);
        acc += rnd<T>(v * v);
      }
    }
  }
  const float m = wave_sum_dpp(acc) / static_cast<float>(d);
  const float r = sqrtf(m + eps);
  if (lane == 0) {
    if (ms) ms[row] = m;
    if (rmsv) rmsv[row] = r;
  }
  const vec* gv = reinterpret_cast<const vec*>(g);
  vec* o = reinterpret_cast<vec*>(out + static_cast<size_t>(row) * d);
  const float inv = rnd<T>(1.0f / r);
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int c = lane + 64 * i;
    if (c < nvec) {
      const vec gg = gv[c];
      vec y;
#pragma unroll
      for (int e = 0; e < E; ++e) {
        const float v = static_cast<float>(xv[i][e]);
        if constexpr (sizeof(T) == 2)
          y[e] = static_cast<T>(rnd<T>(v * inv) * static_cast<float>(gg[e]));
        else
          y[e] = static_cast<T>((v / r) * static_cast<float>(gg[e]));
      }
      o[c] = y;
    }
  }
}

// GELU with the reference's (out, tanh_u) outputs (native/src/gelu.cpp:12-21).
template <typename T>
__global__ __launch_bounds__(256) void gelu_kernel(const T* __restrict__ x, T* __restrict__ out,
                                                   float* __restrict__ tanh_u, size_t n) {
#pragma clang fp contract(off)
  for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; i < n;
       i += static_cast<size_t>(gridDim.x) * blockDim.x) {
    const float v = static_cast<float>(x[i]);
    out[i] = static_cast<T>(gelu_t<T>(v));
    if (tanh_u) {
      if constexpr (sizeof(T) == 2) {
        const float k = static_cast<float>(static_cast<half_t>(0.7978845608028654f));
        const float c = static_cast<float>(static_cast<half_t>(0.044715f));
        float t = rnd<T>(c * v);
        t = rnd<T>(t * v);
        t = rnd<T>(t * v);
        t = rnd<T>(v + t);
        t = rnd<T>(k * t);
        tanh_u[i] = rnd<T>(tanh_h(t));
      } else {
        const float x3 = v * v * v;
        tanh_u[i] = tanhf(0.7978845608028654f * (v + 0.044715f * x3));
      }
    }
  }
}

}  // namespace

int launch_embed(int dt, const int64_t* ids, const void* emb, const void* pos,
                 const int32_t* pos_base, void* out, int B, int S, int d, int V, int P, int* err,
                 hipStream_t st) {
  if (B * S == 0) return 0;
  dim3 grid(B * S), block(256);
  if (dt == F16)
    embed_kernel<half_t><<<grid, block, 0, st>>>(ids, (const half_t*)emb, (const half_t*)pos,
                                                 pos_base, (half_t*)out, S, d, V, P, err);
  else
    embed_kernel<float><<<grid, block, 0, st>>>(ids, (const float*)emb, (const float*)pos,
                                                pos_base, (float*)out, S, d, V, P, err);
  NML_LAUNCHED();
  return 0;
}

int launch_rope(int dt, void* q, void* k, long long kv_stride_b, long long kv_stride_h, int B,
                int H, int S, int dk, const int32_t* pos_base, const int32_t* seq_len,
                const void* cos, const void* sin, int max_len, hipStream_t st) {
  if (B * H * S == 0) return 0;
  NML_REQUIRE(dk % 2 == 0, "rope: head_dim %d must be even", dk);
  const int n = S * (dk / 2);
  dim3 grid((n + 255) / 256, B * H);
  if (dt == F16)
    rope_kernel<half_t><<<grid, 256, 0, st>>>(static_cast<half_t*>(q), static_cast<half_t*>(k),
                                              kv_stride_b, kv_stride_h, H, S, dk, pos_base, seq_len,
                                              static_cast<const half_t*>(cos),
                                              static_cast<const half_t*>(sin), max_len);
  else
    rope_kernel<float><<<grid, 256, 0, st>>>(static_cast<float*>(q), static_cast<float*>(k),
                                             kv_stride_b, kv_stride_h, H, S, dk, pos_base, seq_len,
                                             static_cast<const float*>(cos),
                                             static_cast<const float*>(sin), max_len);
  NML_LAUNCHED();
  return 0;
}

int launch_embed_decode(int dt, const int64_t* tokens, long long tok_stride, const int32_t* pos,
                        const void* emb, const void* posw, void* out, int B, int d, int V, int P,
                        int* err, hipStream_t st) {
  if (B == 0) return 0;
  if (dt == F16)
    embed_decode_kernel<half_t><<<B, 256, 0, st>>>(tokens, tok_stride, pos, (const half_t*)emb,
                                                   (const half_t*)posw, (half_t*)out, d, V, P,
                                                   err);
  else
    embed_decode_kernel<float><<<B, 256, 0, st>>>(tokens, tok_stride, pos, (const float*)emb,
                                                  (const float*)posw, (float*)out, d, V, P, err);
  NML_LAUNCHED();
  return 0;
}

int launch_rmsnorm(int dt, const void* x, const void* g, void* out, float* ms, float* rms,
                   int rows, int d, float eps, hipStream_t st) {
  if (rows == 0) return 0;
  const int E = dt == F16 ? 8 : 4;
  const bool vec_ok = d % E == 0 && ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(g) |
                                      reinterpret_cast<uintptr_t>(out)) & 15) == 0;
  const int nv = (d / E + 63) / 64;
  if (vec_ok && nv <= 8) {
    const int blocks = (rows + 3) / 4;
#define NML_RMS_WAVE(T, NVV) \
  rmsnorm_wave_kernel<T, NVV><<<blocks, 256, 0, st>>>((const T*)x, (const T*)g, (T*)out, ms, rms, rows, d, eps)
    if (dt == F16) {
      if (nv <= 1) NML_RMS_WAVE(half_t, 1);
      else if (nv <= 2) NML_RMS_WAVE(half_t, 2);
      else if (nv <= 4) NML_RMS_WAVE(half_t, 4);
      else NML_RMS_WAVE(half_t, 8);
    } else {
      if (nv <= 1) NML_RMS_WAVE(float, 1);
      else if (nv <= 2) NML_RMS_WAVE(float, 2);
      else if (nv <= 4) NML_RMS_WAVE(float, 4);
      else NML_RMS_WAVE(float, 8);
    }
#undef NML_RMS_WAVE
    NML_LAUNCHED();
    return 0;
  }
  if (dt == F16)
    rmsnorm_kernel<half_t><<<rows, 256, 0, st>>>((const half_t*)x, (const half_t*)g,
                                                 (half_t*)out, ms, rms, d, eps);
  else
    rmsnorm_kernel<float><<<rows, 256, 0, st>>>((const float*)x, (const float*)g, (float*)out,
                                                ms, rms, d, eps);
  NML_LAUNCHED();
  return 0;
}

int launch_gelu(int dt, const void* x, void* out, float* tanh_u, size_t n, hipStream_t st) {
  if (n == 0) return 0;
  size_t blocks = (n + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  if (dt == F16)
    gelu_kernel<half_t><<<blocks, 256, 0, st>>>((const half_t*)x, (half_t*)out, tanh_u, n);
  else
    gelu_kernel<float><<<blocks, 256, 0, st>>>((const float*)x, (float*)out, tanh_u, n);
  NML_LAUNCHED();
  return 0;
}

}  // namespace nml
