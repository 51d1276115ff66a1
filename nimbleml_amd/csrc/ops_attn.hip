// Causal scaled-dot-product attention over the per-layer K/V cache.
//
// Scores follow the reference (kernels/fused_sdpa.py:71-78): s = (q·k) / sqrt(dk),
// then softmax over keys p ≤ query position. In fp16 the score is rounded the
// way the reference's fp16 ops round it (q·k to fp16, then the division by the
// fp16 divisor); the softmax itself runs online in fp32 (flash form), so no
// (S, S) score matrix exists.
//
//  * prefill: one wave per 64 queries of one (sequence, head); K/V tiles of 64
//    keys staged in LDS; online softmax over 16-key sub-tiles.
//  * decode: split-K. One wave per 64-key chunk of one (sequence, head): each lane
//    scores one key, the wave forms the chunk's (max, sum, Σp·v) partial; a
//    combine pass merges the chunks.
#include "kernels.hpp"

namespace nml {

namespace {

constexpr int kTile = 64;

template <typename T, int DK>
__global__ __launch_bounds__(64) void attn_prefill_kernel(AttnArgs a) {
  __shared__ T Ks[kTile][DK];
  __shared__ T Vs[kTile][DK];
  const int lane = threadIdx.x;
  const int bh = blockIdx.y;
  const int b = bh / a.H, h = bh - (bh / a.H) * a.H;
  const int s = blockIdx.x * kTile + lane;
  const int base = a.pos_base ? a.pos_base[b] : 0;
  const int qpos = base + s;
  const int last_s = min(a.S, (blockIdx.x + 1) * kTile) - 1;
  const int kv_end = base + last_s + 1;
  const float scale_t = static_cast<float>(static_cast<T>(a.scale));
  const T* __restrict__ K = static_cast<const T*>(a.k) + b * a.kv_stride_b + h * a.kv_stride_h;
  const T* __restrict__ Vp = static_cast<const T*>(a.v) + b * a.kv_stride_b + h * a.kv_stride_h;

  float q[DK];
  const bool valid = s < a.S;
  {
    const T* qp = static_cast<const T*>(a.q) + ((static_cast<size_t>(bh) * a.S) + (valid ? s : 0)) * DK;
#pragma unroll
    for (int d = 0; d < DK; ++d) q[d] = static_cast<float>(qp[d]);
  }
  float o[DK];
#pragma unroll
  for (int d = 0; d < DK; ++d) o[d] = 0.f;
  float m = -INFINITY, l = 0.f;

  for (int k0 = 0; k0 < kv_end; k0 += kTile) {
    __syncthreads();
    const int key = k0 + lane;
    if (key < kv_end) {
#pragma unroll
      for (int d = 0; d < DK; ++d) {
        Ks[lane][d] = K[static_cast<long long>(key) * DK + d];
        Vs[lane][d] = Vp[static_cast<long long>(key) * DK + d];
      }
    }
    __syncthreads();
    const int nkeys = min(kTile, kv_end - k0);
    for (int j0 = 0; j0 < nkeys; j0 += 16) {
      float sc[16];
      float mloc = -INFINITY;
#pragma unroll
      for (int jj = 0; jj < 16; ++jj) {
        const int kj = j0 + jj;
        float v = -INFINITY;
        if (kj < nkeys && k0 + kj <= qpos) {
          float dot = 0.f;
#pragma unroll
          for (int d = 0; d < DK; ++d) dot += q[d] * static_cast<float>(Ks[kj][d]);
          v = rnd<T>(rnd<T>(dot) / scale_t);
        }
        sc[jj] = v;
        mloc = fmaxf(mloc, v);
      }
      const float mn = fmaxf(m, mloc);
      if (mn == -INFINITY) continue;
      const float alpha = __expf(m - mn);
      l *= alpha;
#pragma unroll
      for (int d = 0; d < DK; ++d) o[d] *= alpha;
#pragma unroll
      for (int jj = 0; jj < 16; ++jj) {
        const float p = expf(sc[jj] - mn);
        if (p != 0.f) {
          l += p;
          const int kj = j0 + jj;
#pragma unroll
          for (int d = 0; d < DK; ++d) o[d] += p * static_cast<float>(Vs[kj][d]);
        }
      }
      m = mn;
    }
  }
  if (valid) {
    const int hd = a.H * DK;
    T* out = static_cast<T*>(a.out) + (static_cast<size_t>(b) * a.S + s) * hd + h * DK;
    const float inv = 1.f / l;
#pragma unroll
    for (int d = 0; d < DK; ++d) out[d] = static_cast<T>(o[d] * inv);
  }
}

template <typename T, int DK>
__global__ __launch_bounds__(64) void attn_decode_kernel(AttnArgs a, const int32_t* __restrict__ pos,
                                                         int max_chunks, float* __restrict__ part) {
  const int lane = threadIdx.x;
  const int c = blockIdx.x, bh = blockIdx.y;
  const int b = bh / a.H, h = bh - (bh / a.H) * a.H;
  const int len = pos[b] + 1;
  const int k0 = c * kTile;
  float* pp = part + (static_cast<size_t>(bh) * max_chunks + c) * (DK + 2);
  if (k0 >= len) return;  // the combine pass only reads chunks below len
  const float scale_t = static_cast<float>(static_cast<T>(a.scale));
  const T* __restrict__ K = static_cast<const T*>(a.k) + b * a.kv_stride_b + h * a.kv_stride_h;
  const T* __restrict__ Vp = static_cast<const T*>(a.v) + b * a.kv_stride_b + h * a.kv_stride_h;
  const T* __restrict__ qp = static_cast<const T*>(a.q) + static_cast<size_t>(bh) * DK;

  const int key = k0 + lane;
  float sc = -INFINITY;
  if (key < len) {
    const T* kr = K + static_cast<long long>(key) * DK;
    float dot = 0.f;
#pragma unroll
    for (int d = 0; d < DK; ++d) dot += static_cast<float>(qp[d]) * static_cast<float>(kr[d]);
    sc = rnd<T>(rnd<T>(dot) / scale_t);
  }
  const float mx = wave_max(sc);
  const float p = (key < len) ? expf(sc - mx) : 0.f;
  const float l = wave_sum(p);
  const int nkeys = min(kTile, len - k0);
  constexpr int DPL = (DK + 63) / 64;  // output dims per lane
#pragma unroll
  for (int t = 0; t < DPL; ++t) {
    const int d = lane + 64 * t;
    float acc = 0.f;
    for (int j = 0; j < nkeys; ++j) {
      const float pj = __shfl(p, j, 64);
      if (d < DK) acc += pj * static_cast<float>(Vp[static_cast<long long>(k0 + j) * DK + d]);
    }
    if (d < DK) pp[2 + d] = acc;
  }
  if (lane == 0) {
    pp[0] = mx;
    pp[1] = l;
  }
}

template <typename T, int DK>
__global__ __launch_bounds__(64) void attn_combine_kernel(AttnArgs a, const int32_t* __restrict__ pos,
                                                          int max_chunks, const float* __restrict__ part) {
  const int lane = threadIdx.x;
  const int bh = blockIdx.x;
  const int b = bh / a.H, h = bh - (bh / a.H) * a.H;
  const int len = pos[b] + 1;
  const int nc = (len + kTile - 1) / kTile;
  const float* pb = part + static_cast<size_t>(bh) * max_chunks * (DK + 2);
  float M = -INFINITY;
  for (int c = 0; c < nc; ++c) M = fmaxf(M, pb[c * (DK + 2)]);
  float den = 0.f;
  for (int c = 0; c < nc; ++c) den += __expf(pb[c * (DK + 2)] - M) * pb[c * (DK + 2) + 1];
  const float inv = 1.f / den;
  T* out = static_cast<T*>(a.out) + static_cast<size_t>(b) * a.H * DK + h * DK;
  for (int d = lane; d < DK; d += 64) {
    float num = 0.f;
    for (int c = 0; c < nc; ++c) num += __expf(pb[c * (DK + 2)] - M) * pb[c * (DK + 2) + 2 + d];
    out[d] = static_cast<T>(num * inv);
  }
}

template <typename T, int DK>
int prefill_typed(const AttnArgs& a, hipStream_t st) {
  dim3 grid((a.S + kTile - 1) / kTile, a.B * a.H);
  attn_prefill_kernel<T, DK><<<grid, 64, 0, st>>>(a);
  NML_LAUNCHED();
  return 0;
}

template <typename T, int DK>
int decode_typed(const AttnArgs& a, const int32_t* pos, int max_len, float* part, hipStream_t st) {
  const int max_chunks = (max_len + kTile - 1) / kTile;
  dim3 grid(max_chunks, a.B * a.H);
  attn_decode_kernel<T, DK><<<grid, 64, 0, st>>>(a, pos, max_chunks, part);
  NML_LAUNCHED();
  attn_combine_kernel<T, DK><<<a.B * a.H, 64, 0, st>>>(a, pos, max_chunks, part);
  NML_LAUNCHED();
  return 0;
}

#define NML_DK_SWITCH(dk, FN, ...)                                  \
  switch (dk) {                                                     \
    case 8: return FN<T, 8>(__VA_ARGS__);                           \
    case 16: return FN<T, 16>(__VA_ARGS__);                         \
    case 32: return FN<T, 32>(__VA_ARGS__);                         \
    case 64: return FN<T, 64>(__VA_ARGS__);                         \
    case 128: return FN<T, 128>(__VA_ARGS__);                       \
    default: set_error("attention: head_dim %d unsupported (8, 16, 32, 64, 128)", dk); \
      return -1;                                                    \
  }

template <typename T>
int prefill_dk(const AttnArgs& a, hipStream_t st) {
  NML_DK_SWITCH(a.dk, prefill_typed, a, st);
}

template <typename T>
int decode_dk(const AttnArgs& a, const int32_t* pos, int max_len, float* part, hipStream_t st) {
  NML_DK_SWITCH(a.dk, decode_typed, a, pos, max_len, part, st);
}

}  // namespace

size_t attention_decode_workspace(int B, int H, int dk, int max_len) {
  const size_t chunks = (max_len + kTile - 1) / kTile;
  return static_cast<size_t>(B) * H * chunks * (dk + 2) * sizeof(float);
}

int launch_attention_prefill(int dt, const AttnArgs& a, hipStream_t st) {
  if (a.B * a.S == 0) return 0;
  return dt == F16 ? prefill_dk<half_t>(a, st) : prefill_dk<float>(a, st);
}

int launch_attention_decode(int dt, const AttnArgs& a, const int32_t* pos, int max_len, float* part,
                            hipStream_t st) {
  if (a.B == 0) return 0;
  NML_REQUIRE(max_len > 0, "attention decode: max_len must be positive");
  return dt == F16 ? decode_dk<half_t>(a, pos, max_len, part, st)
                   : decode_dk<float>(a, pos, max_len, part, st);
}

}  // namespace nml
