// Shared definitions for the gfx950 (CDNA4) kernels and the C-ABI.
//
// Every C-ABI entry point returns 0 on success and -1 on failure; the failure
// text is kept per thread and read with nml_last_error(). Launches go to the
// library stream (nml_get_stream / nml_set_stream), asynchronously.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace nml {

typedef _Float16 half_t;
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

enum DType : int { F32 = 0, F16 = 1 };

inline size_t dtype_size(int dt) { return dt == F16 ? 2 : 4; }

// Per-thread error text (host side).
void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
hipStream_t stream();
hipStream_t stream2();  // a second stream for forked work, joined back by events
bool is_stream2(hipStream_t s);

constexpr int kWave = 64;

// ----------------------------------------------------------------- device math
// Rounding helpers: round a float to the storage type T and back. For
// T = half this reproduces one NumPy fp16 op (float compute, one rounding).
template <typename T>
__device__ __forceinline__ float rnd(float x) {
  return static_cast<float>(static_cast<T>(x));
}

template <typename T>
__device__ __forceinline__ float ld(const T* p) {
  return static_cast<float>(*p);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// Wave reductions on the VALU data-parallel-primitive path (DPP lane moves, ~4 cycles
// each) instead of LDS-crossbar shuffles (~100 cycles each): butterflies xor 1 and xor 2
// inside quads, then half-row and row mirrors give every lane its 16-lane row value,
// and the four rows are combined from lanes 0, 16, 32, 48 (a wave-uniform result).
template <int CTRL>
__device__ __forceinline__ float dpp_move(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
constexpr int kDppXor1 = 0xB1;         // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;         // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141;  // row_half_mirror
constexpr int kDppMirror = 0x140;      // row_mirror

__device__ __forceinline__ float lane_f(float v, int l) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}

__device__ __forceinline__ float wave_sum_dpp(float v) {
  v += dpp_move<kDppXor1>(v);
  v += dpp_move<kDppXor2>(v);
  v += dpp_move<kDppHalfMirror>(v);
  v += dpp_move<kDppMirror>(v);
  return (lane_f(v, 0) + lane_f(v, 16)) + (lane_f(v, 32) + lane_f(v, 48));
}

__device__ __forceinline__ float wave_max_dpp(float v) {
  v = fmaxf(v, dpp_move<kDppXor1>(v));
  v = fmaxf(v, dpp_move<kDppXor2>(v));
  v = fmaxf(v, dpp_move<kDppHalfMirror>(v));
  v = fmaxf(v, dpp_move<kDppMirror>(v));
  return fmaxf(fmaxf(lane_f(v, 0), lane_f(v, 16)), fmaxf(lane_f(v, 32), lane_f(v, 48)));
}

// Sum over the 16 lanes of each row (lanes 16k..16k+15), the same value in every lane.
__device__ __forceinline__ float row16_sum_dpp(float v) {
  v += dpp_move<kDppXor1>(v);
  v += dpp_move<kDppXor2>(v);
  v += dpp_move<kDppHalfMirror>(v);
  return v + dpp_move<kDppMirror>(v);
}

// Sum over the 4 lanes of each quad (lanes 4k..4k+3), in every lane of the quad.
__device__ __forceinline__ float quad_sum_dpp(float v) {
  v += dpp_move<kDppXor1>(v);
  return v + dpp_move<kDppXor2>(v);
}

__device__ __forceinline__ double wave_sum_d(double v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Block-wide sum for blockDim.x a multiple of 64 (≤ 1024); `red` holds 16 floats.
__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wave_sum(v);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
  __syncthreads();
  if (lane == 0) red[w] = v;
  __syncthreads();
  float t = 0.f;
  for (int i = 0; i < nw; ++i) t += red[i];
  return t;
}

// tanh of an fp16 value t, as accurate as its rounding to fp16 needs: below |t| = 0.3 an
// odd polynomial, t·p(t²) with p a least-squares fit of tanh(a)/a on a² ∈ [0, 0.09]
// (relative error below 1e-12 in exact arithmetic); above, 1 − 2/(e^{2|t|} + 1) with the
// hardware exp2 and reciprocal. Rounded to fp16 it equals NumPy's float16 tanh (the
// reference's fp16 GELU, kernels/fused_gelu.py:67-69) on every fp16 input when evaluated
// in float32 — and still on all but at most 3 of them with the exp and the reciprocal
// each off by up to two ulps — at a fraction of tanhf's cost.
__device__ __forceinline__ float tanh_h(float t) {
  const float a = fabsf(t), s = a * a;
  float p = -0.0079558f;
  p = p * s + 0.02177956f;
  p = p * s - 0.0539641f;
  p = p * s + 0.13333325f;
  p = p * s - 0.33333333f;
  p = p * s + 1.0f;
  const float e = __builtin_amdgcn_exp2f(a * 2.8853900817779268f);  // e^{2a}
  const float r = 1.0f - 2.0f * __builtin_amdgcn_rcpf(e + 1.0f);
  return copysignf(a < 0.3f ? p * a : r, t);
}

// GELU, tanh form: 0.5·x·(1 + tanh(√(2/π)·(x + 0.044715·x³))).
// fp32: the operation order of the reference's native kernel
// (native/src/gelu.cpp:15-19). fp16: the reference evaluates the same formula
// as NumPy fp16 ufuncs (kernels/fused_gelu.py:67-69), Python constants taken
// as fp16, left to right, one rounding per op — reproduced op by op here.
__device__ __forceinline__ float gelu_f32(float x) {
#pragma clang fp contract(off)
  const float x3 = x * x * x;
  const float tu = tanhf(0.7978845608028654f * (x + 0.044715f * x3));
  return 0.5f * x * (1.0f + tu);
}

__device__ __forceinline__ float gelu_f16(float x) {
#pragma clang fp contract(off)
  const float k = static_cast<float>(static_cast<half_t>(0.7978845608028654f));
  const float c = static_cast<float>(static_cast<half_t>(0.044715f));
  float t = rnd<half_t>(c * x);
  t = rnd<half_t>(t * x);
  t = rnd<half_t>(t * x);
  t = rnd<half_t>(x + t);
  t = rnd<half_t>(k * t);
  const float tu = rnd<half_t>(tanh_h(t));
  const float a = rnd<half_t>(0.5f * x);
  const float b = rnd<half_t>(1.0f + tu);
  return rnd<half_t>(a * b);
}

// gelu_f16 on 8 fp16 values at once. A product or sum of two fp16 values taken in fp32
// and rounded to fp16 equals the correctly rounded fp16 operation (fp32 carries 24 ≥
// 2·11 + 2 significand bits, so the double rounding is innocuous), so the native fp16
// operations here (packed, two per instruction) give gelu_f16's values; the tanh is
// tanh_h as there.
__device__ __forceinline__ half8 gelu8_f16(half8 x) {
#pragma clang fp contract(off)
  const half_t k = static_cast<half_t>(0.7978845608028654f);
  const half_t c = static_cast<half_t>(0.044715f);
  half8 t = x * c;
  t = t * x;
  t = t * x;
  t = x + t;
  t = t * k;
  half8 tu;
#pragma unroll
  for (int e = 0; e < 8; ++e) tu[e] = static_cast<half_t>(tanh_h(static_cast<float>(t[e])));
  const half8 a = x * static_cast<half_t>(0.5f);
  const half8 b = tu + static_cast<half_t>(1.0f);
  return a * b;
}

template <typename T>
__device__ __forceinline__ float gelu_t(float x);
template <>
__device__ __forceinline__ float gelu_t<float>(float x) { return gelu_f32(x); }
template <>
__device__ __forceinline__ float gelu_t<half_t>(float x) { return gelu_f16(x); }

}  // namespace nml

#define NML_HIP(call)                                                              \
  do {                                                                             \
    hipError_t e_ = (call);                                                        \
    if (e_ != hipSuccess) {                                                        \
      nml::set_error("%s failed: %s (%s:%d)", #call, hipGetErrorString(e_),         \
                     __FILE__, __LINE__);                                          \
      return -1;                                                                   \
    }                                                                              \
  } while (0)

#define NML_REQUIRE(cond, ...)                                                     \
  do {                                                                             \
    if (!(cond)) {                                                                 \
      nml::set_error(__VA_ARGS__);                                                 \
      return -1;                                                                   \
    }                                                                              \
  } while (0)

// Check the launch that was just issued.
#define NML_LAUNCHED()                                                             \
  do {                                                                             \
    hipError_t e_ = hipGetLastError();                                             \
    if (e_ != hipSuccess) {                                                        \
      nml::set_error("kernel launch failed: %s (%s:%d)", hipGetErrorString(e_),     \
                     __FILE__, __LINE__);                                          \
      return -1;                                                                   \
    }                                                                              \
  } while (0)

#define NML_TRY(expr)                                                              \
  do {                                                                             \
    if ((expr) != 0) return -1;                                                    \
  } while (0)
