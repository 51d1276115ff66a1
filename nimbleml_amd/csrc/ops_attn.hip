// Causal scaled-dot-product attention over the per-layer K/V cache.
//
// Scores follow the reference (kernels/fused_sdpa.py:71-78): s = (q·k) / sqrt(dk),
// then softmax over keys p ≤ query position. In fp16 the score is rounded the
// way the reference's fp16 ops round it (q·k to fp16, then the division by the
// fp16 divisor); the softmax itself runs online in fp32 (flash form), so no
// (S, S) score matrix exists.
//
//  * prefill, fp16 head dim 64/128: MFMA flash attention, 128 queries per workgroup,
//    64-key K/V tiles in LDS — attn_prefill_pipe_kernel (fp32 scores, software-pipelined
//    over the tiles) where no statistics are kept, attn_prefill_mfma_kernel (fp16-rounded
//    scores, statistics for the backward) otherwise;
//    fp32 head dim 64/128: attn_prefill_f32_mfma; head dims 8/16/32 (and the non-causal
//    masked form): attn_prefill_kernel, one wave per 64 queries, scalar; any other head
//    dim ≤ 256: attn_prefill_quad_kernel, four lanes per query.
//  * decode, head dim 32/64/128/256: attn_decode_group_kernel — split-K in one launch:
//    each workgroup scores a group of 64-key chunks of one (sequence, head) and publishes
//    its (max, Σp, Σp·v) as flagged slots; the last workgroup of the (sequence, head)
//    merges them. Other head dims ≤ 256: attn_decode_small_kernel + attn_combine_kernel.
#include <cstdlib>
#include <type_traits>

#include "kernels.hpp"

namespace nml {

namespace {

constexpr int kTile = 64;
constexpr int kCombineMax = 1024;  // chunks of one (row, head): max_seq_len ≤ 65536


template <typename T, int DK>
__global__ __launch_bounds__(64) void attn_prefill_kernel(AttnArgs a) {
  __shared__ T Ks[kTile][DK];
  __shared__ T Vs[kTile][DK];
  const int lane = threadIdx.x;
  const int bh = blockIdx.y;
  const int b = bh / a.H, h = bh - (bh / a.H) * a.H;
  const int s = blockIdx.x * kTile + lane;
  const int S = a.seq_len ? a.seq_len[b] : a.S;
  if (static_cast<int>(blockIdx.x) * kTile >= S) return;  // past a ragged sequence's end
  const int base = a.pos_base ? a.pos_base[b] : 0;
  const int qpos = base + s;
  const int last_s = min(S, (blockIdx.x + 1) * kTile) - 1;
  const int kv_end = a.full ? S : base + last_s + 1;
  const float scale_t = static_cast<float>(static_cast<T>(a.scale));
  const T* __restrict__ K = static_cast<const T*>(a.k) + b * a.kv_stride_b + h * a.kv_stride_h;
  const T* __restrict__ Vp = static_cast<const T*>(a.v) + b * a.kv_stride_b + h * a.kv_stride_h;

  float q[DK];
  const bool valid = s < S;
  // row s of the additive mask (row 0 for the idle lanes past S)
  const T* __restrict__ mrow =
      a.mask ? static_cast<const T*>(a.mask) + static_cast<size_t>(valid ? s : 0) * S : nullptr;
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
        if (kj < nkeys && (a.full || k0 + kj <= qpos)) {
          float dot = 0.f;
#pragma unroll
          for (int d = 0; d < DK; ++d) dot += q[d] * static_cast<float>(Ks[kj][d]);
          v = rnd<T>(rnd<T>(dot) / scale_t);
          if (mrow) v = rnd<T>(v + static_cast<float>(mrow[k0 + kj]));
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
    const size_t row = (a.row_start ? a.row_start[b] : static_cast<size_t>(b) * a.S) + s;
    T* out = static_cast<T*>(a.out) + row * hd + h * DK;
    const float inv = 1.f / l;
#pragma unroll
    for (int d = 0; d < DK; ++d) out[d] = static_cast<T>(o[d] * inv);
    if (a.lse) a.lse[static_cast<size_t>(bh) * a.S + s] = m + logf(l);
    if (a.m_out) {
      a.m_out[static_cast<size_t>(bh) * a.S + s] = m;
      a.l_out[static_cast<size_t>(bh) * a.S + s] = l;
    }
  }
}

// Prefill for any head dim up to 4·DPL (the runtime a.dk: 96, 80, 256, ...), the
// attn_prefill_kernel semantics (same score roundings, mask, ragged rows and statistics)
// with four lanes per query: lane `sub` of a query's quad owns dims sub + 4i, so a lane
// keeps DPL query and output values in registers (at dk 256, 64 + 64 instead of 512). A
// workgroup takes 64 queries (16 per wave) and walks key tiles of KT rows staged in LDS,
// zero-padded to 4·DPL columns; a score is the quad's four partial dot products summed
// by DPP lane moves.
template <typename T, int DPL>
__global__ __launch_bounds__(256) void attn_prefill_quad_kernel(AttnArgs a) {
  constexpr int QW = 64, DKP = 4 * DPL, KT = DPL >= 64 ? 16 : 32;
  __shared__ T Ks[KT][DKP];
  __shared__ T Vs[KT][DKP];
  const int tid = threadIdx.x, sub = tid & 3;
  const int dk = a.dk;
  const int bh = blockIdx.y;
  const int b = bh / a.H, h = bh - (bh / a.H) * a.H;
  const int s = blockIdx.x * QW + (tid >> 2);
  const int S = a.seq_len ? a.seq_len[b] : a.S;
  if (static_cast<int>(blockIdx.x) * QW >= S) return;  // past a ragged sequence's end
  const int base = a.pos_base ? a.pos_base[b] : 0;
  const int qpos = base + s;
  const int last_s = min(S, (blockIdx.x + 1) * QW) - 1;
  const int kv_end = a.full ? S : base + last_s + 1;
  const float scale_t = static_cast<float>(static_cast<T>(a.scale));
  const T* __restrict__ K = static_cast<const T*>(a.k) + b * a.kv_stride_b + h * a.kv_stride_h;
  const T* __restrict__ Vp = static_cast<const T*>(a.v) + b * a.kv_stride_b + h * a.kv_stride_h;
  const bool valid = s < S;
  const T* __restrict__ mrow =
      a.mask ? static_cast<const T*>(a.mask) + static_cast<size_t>(valid ? s : 0) * S : nullptr;
  float q[DPL], o[DPL];
  {
    const T* qp = static_cast<const T*>(a.q) + ((static_cast<size_t>(bh) * a.S) + (valid ? s : 0)) * dk;
#pragma unroll
    for (int i = 0; i < DPL; ++i) {
      const int d = sub + 4 * i;
      q[i] = d < dk ? static_cast<float>(qp[d]) : 0.f;
      o[i] = 0.f;
    }
  }
  float m = -INFINITY, l = 0.f;
  for (int k0 = 0; k0 < kv_end; k0 += KT) {
    __syncthreads();  // the previous tile's readers are done
    for (int e = tid; e < KT * DKP; e += 256) {
      const int r = e / DKP, c = e - (e / DKP) * DKP, key = k0 + r;
      const bool in = key < kv_end && c < dk;
      Ks[r][c] = in ? K[static_cast<long long>(key) * dk + c] : static_cast<T>(0.f);
      Vs[r][c] = in ? Vp[static_cast<long long>(key) * dk + c] : static_cast<T>(0.f);
    }
    __syncthreads();
    const int nkeys = min(KT, kv_end - k0);
    for (int j0 = 0; j0 < nkeys; j0 += 16) {
      float sc[16];
      float mloc = -INFINITY;
#pragma unroll
      for (int jj = 0; jj < 16; ++jj) {
        const int kj = j0 + jj;  // < KT: rows past nkeys are zero-filled
        float dot = 0.f;
#pragma unroll
        for (int i = 0; i < DPL; ++i) dot += q[i] * static_cast<float>(Ks[kj][sub + 4 * i]);
        dot = quad_sum_dpp(dot);  // every lane of the quad: no divergence before this
        float v = -INFINITY;
        if (kj < nkeys && (a.full || k0 + kj <= qpos)) {
          v = rnd<T>(rnd<T>(dot) / scale_t);
          if (mrow) v = rnd<T>(v + static_cast<float>(mrow[k0 + kj]));
        }
        sc[jj] = v;
        mloc = fmaxf(mloc, v);
      }
      const float mn = fmaxf(m, mloc);
      if (mn == -INFINITY) continue;
      const float alpha = __expf(m - mn);
      l *= alpha;
#pragma unroll
      for (int i = 0; i < DPL; ++i) o[i] *= alpha;
#pragma unroll
      for (int jj = 0; jj < 16; ++jj) {
        const float p = expf(sc[jj] - mn);
        if (p != 0.f) {
          l += p;
          const int kj = j0 + jj;
#pragma unroll
          for (int i = 0; i < DPL; ++i) o[i] += p * static_cast<float>(Vs[kj][sub + 4 * i]);
        }
      }
      m = mn;
    }
  }
  if (valid) {
    const size_t row = (a.row_start ? a.row_start[b] : static_cast<size_t>(b) * a.S) + s;
    T* out = static_cast<T*>(a.out) + row * a.H * dk + h * dk;
    const float inv = 1.f / l;
#pragma unroll
    for (int i = 0; i < DPL; ++i) {
      const int d = sub + 4 * i;
      if (d < dk) out[d] = static_cast<T>(o[i] * inv);
    }
    if (sub == 0) {
      if (a.lse) a.lse[static_cast<size_t>(bh) * a.S + s] = m + logf(l);
      if (a.m_out) {
        a.m_out[static_cast<size_t>(bh) * a.S + s] = m;
        a.l_out[static_cast<size_t>(bh) * a.S + s] = l;
      }
    }
  }
}

// 16-byte loads of 8 consecutive elements.
template <typename T>
__device__ __forceinline__ void ld8(const T* p, float (&o)[8]) {
  if constexpr (sizeof(T) == 2) {
    const half8 v = *reinterpret_cast<const half8*>(p);
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = static_cast<float>(v[e]);
  } else {
    const floatx4 x = *reinterpret_cast<const floatx4*>(p);
    const floatx4 y = *reinterpret_cast<const floatx4*>(p + 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      o[e] = x[e];
      o[4 + e] = y[e];
    }
  }
}

// 8 consecutive elements kept in their storage type (half: one 16-byte register
// quad), widened where they are used.
template <typename T>
struct Raw8;
template <>
struct Raw8<half_t> {
  half8 v;
  __device__ __forceinline__ void load(const half_t* p) { v = *reinterpret_cast<const half8*>(p); }
  __device__ __forceinline__ float at(int e) const { return static_cast<float>(v[e]); }
};
template <>
struct Raw8<float> {
  floatx4 x, y;
  __device__ __forceinline__ void load(const float* p) {
    x = *reinterpret_cast<const floatx4*>(p);
    y = *reinterpret_cast<const floatx4*>(p + 4);
  }
  __device__ __forceinline__ float at(int e) const { return e < 4 ? x[e] : y[e - 4]; }
};

// Decode attention for head dims ≥ 32, one launch: a 256-lane workgroup takes a group
// of G 64-key chunks of one (row, head) — their K rows are loaded up front and their V
// rows once the scores are formed (clamped into [0, len), the clamped ones never used;
// K and V are never held together, which keeps the kernel at ≤ 72 registers: seven
// workgroups per CU, so a batched step's groups are all resident at once) — scores
// every key with 4 lanes per key (DK/4 dims each), takes the group's max and Σp with
// one block reduction each, and P·V with each lane owning 8 dims of a key subset
// (C4, hd 64: 21.9 → 21.0 µs a layer against the K and V both loaded up front). Every group
// but the last of its (row, head) publishes (max, Σp, Σp·v) as flagged 64-bit slots
// (1 << 32 | value, relaxed device-scope stores, no fences) and exits. The last group
// — later in dispatch order than its siblings (x is the fastest grid index), so its
// bounded wait always ends — waits for their slots, merges them with its own partial
// (softmax rescaling, attention.py:140-142 over the concatenated keys), writes the
// head's output and returns the slots to zero for the next launch.
// slots per group partial: DK + 2 rounded up to whole 128-byte lines
constexpr int dec_slots(int dk) { return (dk + 2 + 15) / 16 * 16; }

template <typename T, int DK>
constexpr int dec_groups() {  // chunks per group: K/V registers bounded
  return DK * static_cast<int>(sizeof(T)) <= 128 ? 4 : DK * static_cast<int>(sizeof(T)) <= 256 ? 2 : 1;
}

template <typename T, int DK, int G>
__global__ __launch_bounds__(256) void attn_decode_group_kernel(AttnArgs a, const int32_t* __restrict__ pos,
                                                                int max_groups,
                                                                unsigned long long* __restrict__ part) {
#pragma clang fp contract(off)
  typedef unsigned long long u64;
  constexpr int CH = kTile, KG = CH * G, DPT = DK / 4, DG = DK / 8, NKS = 256 / DG, KPT = CH / NKS;
  constexpr int PS = dec_slots(DK);
  static_assert(DK >= 32 && KPT >= 1, "decode group shape");
  __shared__ float s_q[DK], s_p[KG], s_red[16];
  __shared__ float s_o[NKS][DK + 1];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int grp = blockIdx.x, bh = blockIdx.y;
  const int b = bh / a.H, h = bh - (bh / a.H) * a.H;
  const int len = pos[b] + 1;
  const int k0 = grp * KG;
  if (k0 >= len) return;  // whole workgroup: groups at or past len do nothing
  const int ng = (len + KG - 1) / KG;
  const T* __restrict__ K = static_cast<const T*>(a.k) + b * a.kv_stride_b + h * a.kv_stride_h;
  const T* __restrict__ Vp = static_cast<const T*>(a.v) + b * a.kv_stride_b + h * a.kv_stride_h;
  const float scale_t = static_cast<float>(static_cast<T>(a.scale));
  const int qq = tid & 3, dg = tid % DG, ks = tid / DG;
  // K/V stay in their storage type in registers (half the registers of widened copies,
  // so more workgroups per CU keep loads in flight)
  Raw8<T> kr[G][DPT / 8];
  Raw8<T> vr[G][KPT];
#pragma unroll
  for (int j = 0; j < G; ++j) {
    const int key = k0 + j * CH + (tid >> 2);
    const int keyc = key < len ? key : len - 1;
#pragma unroll
    for (int e = 0; e < DPT / 8; ++e) kr[j][e].load(K + static_cast<long long>(keyc) * DK + qq * DPT + e * 8);
  }
  if (tid < DK) s_q[tid] = static_cast<float>(static_cast<const T*>(a.q)[static_cast<size_t>(bh) * DK + tid]);
  __syncthreads();
  float sc[G];
  float mx = -INFINITY;
#pragma unroll
  for (int j = 0; j < G; ++j) {
    float dot = 0.f;
#pragma unroll
    for (int e = 0; e < DPT; ++e) dot += s_q[qq * DPT + e] * kr[j][e / 8].at(e % 8);
    dot = quad_sum_dpp(dot);
    const bool valid = k0 + j * CH + (tid >> 2) < len;
    sc[j] = valid ? rnd<T>(rnd<T>(dot) / scale_t) : -INFINITY;
    mx = fmaxf(mx, sc[j]);
  }
  mx = wave_max_dpp(mx);
  if (lane == 0) s_red[wave] = mx;
  __syncthreads();
#pragma unroll
  for (int j = 0; j < G; ++j)
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
      const int vk = k0 + j * CH + ks + i * NKS;
      vr[j][i].load(Vp + static_cast<long long>(vk < len ? vk : len - 1) * DK + dg * 8);
    }
  mx = fmaxf(fmaxf(s_red[0], s_red[1]), fmaxf(s_red[2], s_red[3]));
  float lsum = 0.f;
#pragma unroll
  for (int j = 0; j < G; ++j) {
    const float p = expf(sc[j] - mx);  // exp(-inf) = 0 for keys past len
    if (qq == 0) {
      s_p[j * CH + (tid >> 2)] = p;
      lsum += p;
    }
  }
  lsum = wave_sum_dpp(lsum);
  if (lane == 0) s_red[4 + wave] = lsum;
  __syncthreads();
  const float l = (s_red[4] + s_red[5]) + (s_red[6] + s_red[7]);
  float o[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = 0.f;
#pragma unroll
  for (int j = 0; j < G; ++j)
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
      const int jj = j * CH + ks + i * NKS;
      if (k0 + jj < len) {
        const float pj = s_p[jj];
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] += pj * vr[j][i].at(e);
      }
    }
#pragma unroll
  for (int e = 0; e < 8; ++e) s_o[ks][dg * 8 + e] = o[e];
  __syncthreads();
  u64* const pb = part + static_cast<size_t>(bh) * max_groups * PS;
  const u64 flag = 1ull << 32;
  float own = 0.f;
  if (tid < DK)
    for (int k2 = 0; k2 < NKS; ++k2) own += s_o[k2][tid];
  if (grp != ng - 1) {  // publish this group's partial and leave
    // (max, Σp) from the first lane past the head's dims; at DK 256 (no such lane) lane 0
    constexpr int kStatLane = DK < 256 ? DK : 0;
    if (tid < DK)
      __hip_atomic_store(pb + grp * PS + 2 + tid, flag | __float_as_uint(own), __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
    if (tid == kStatLane) {
      __hip_atomic_store(pb + grp * PS, flag | __float_as_uint(mx), __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(pb + grp * PS + 1, flag | __float_as_uint(l), __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
    }
    return;
  }
  // The last group of (b, h) — dispatched after its siblings, which wait on nothing —
  // waits (bounded) for their slots, 8 groups' slots in flight at a time, and merges
  // them in group order, its own partial last.
  if (tid < DK) {
    constexpr int NB = 8;
    float mg[NB], lg[NB], og[NB];
    float M = -INFINITY, den = 0.f, num = 0.f;
    const int np = ng - 1;
    for (int g0 = 0; g0 < np; g0 += NB) {
      u64 vm[NB], vl[NB], vo[NB];
      const u64 ok = 1ull << 32;
#pragma unroll
      for (int j = 0; j < NB; ++j) {
        const bool in = g0 + j < np;
        u64* sl = pb + (g0 + j) * PS;
        vm[j] = in ? __hip_atomic_load(sl, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : ok;
        vl[j] = in ? __hip_atomic_load(sl + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : ok;
        vo[j] = in ? __hip_atomic_load(sl + 2 + tid, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : ok;
      }
      for (unsigned spins = 0; spins < (1u << 22); ++spins) {
        bool all = true;
#pragma unroll
        for (int j = 0; j < NB; ++j) all = all && (vm[j] >> 32) && (vl[j] >> 32) && (vo[j] >> 32);
        if (all) break;
        __builtin_amdgcn_s_sleep(1);
#pragma unroll
        for (int j = 0; j < NB; ++j) {
          u64* sl = pb + (g0 + j) * PS;
          if (!(vm[j] >> 32)) vm[j] = __hip_atomic_load(sl, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          if (!(vl[j] >> 32)) vl[j] = __hip_atomic_load(sl + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          if (!(vo[j] >> 32))
            vo[j] = __hip_atomic_load(sl + 2 + tid, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      }
#pragma unroll
      for (int j = 0; j < NB; ++j) {
        mg[j] = __uint_as_float(static_cast<uint32_t>(vm[j]));
        lg[j] = __uint_as_float(static_cast<uint32_t>(vl[j]));
        og[j] = __uint_as_float(static_cast<uint32_t>(vo[j]));
      }
      // online merge over this batch of groups (in group order)
#pragma unroll
      for (int j = 0; j < NB; ++j) {
        if (g0 + j >= np) break;
        const float Mn = fmaxf(M, mg[j]);
        const float c = expf(M - Mn), w = expf(mg[j] - Mn);
        den = den * c + w * lg[j];
        num = num * c + w * og[j];
        M = Mn;
      }
    }
    {  // this group
      const float Mn = fmaxf(M, mx);
      const float c = expf(M - Mn), w = expf(mx - Mn);
      den = den * c + w * l;
      num = num * c + w * own;
    }
    T* out = static_cast<T*>(a.out) + static_cast<size_t>(b) * a.H * DK + h * DK;
    out[tid] = static_cast<T>(num * (1.f / den));
  }
  __syncthreads();  // every read of the slots done before they are cleared
  for (int i = tid; i < (ng - 1) * PS; i += 256)
    __hip_atomic_store(pb + i, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Decode attention for head dims outside the group kernel's set (8, 16 and any dk that
// is not 32, 64, 128 or 256; runtime a.dk ≤ 256): one wave per 64-key chunk, lane j
// scores key k0 + j, then P·V with each lane owning up to four output dims; the chunk's
// (max, Σp, Σp·v) go to `part` for attn_combine_kernel.
template <typename T>
__global__ __launch_bounds__(64) void attn_decode_small_kernel(AttnArgs a, const int32_t* __restrict__ pos,
                                                         int max_chunks, float* __restrict__ part) {
  const int lane = threadIdx.x;
  const int c = blockIdx.x, bh = blockIdx.y;
  const int b = bh / a.H, h = bh - (bh / a.H) * a.H;
  const int dk = a.dk;
  const int len = pos[b] + 1;
  const int k0 = c * kTile;
  float* pp = part + (static_cast<size_t>(bh) * max_chunks + c) * (dk + 2);
  if (k0 >= len) return;  // the combine pass only reads chunks below len
  const float scale_t = static_cast<float>(static_cast<T>(a.scale));
  const T* __restrict__ K = static_cast<const T*>(a.k) + b * a.kv_stride_b + h * a.kv_stride_h;
  const T* __restrict__ Vp = static_cast<const T*>(a.v) + b * a.kv_stride_b + h * a.kv_stride_h;
  const T* __restrict__ qp = static_cast<const T*>(a.q) + static_cast<size_t>(bh) * dk;

  const int key = k0 + lane;
  float sc = -INFINITY;
  if (key < len) {
    const T* kr = K + static_cast<long long>(key) * dk;
    float dot = 0.f;
    for (int d = 0; d < dk; ++d) dot += static_cast<float>(qp[d]) * static_cast<float>(kr[d]);
    sc = rnd<T>(rnd<T>(dot) / scale_t);
  }
  const float mx = wave_max(sc);
  const float p = (key < len) ? expf(sc - mx) : 0.f;
  const float l = wave_sum(p);
  const int nkeys = min(kTile, len - k0);
  constexpr int DPL = 4;  // output dims per lane: dk ≤ 256
#pragma unroll
  for (int t = 0; t < DPL; ++t) {
    const int d = lane + 64 * t;
    float acc = 0.f;
    for (int j = 0; j < nkeys; ++j) {
      const float pj = __shfl(p, j, 64);
      if (d < dk) acc += pj * static_cast<float>(Vp[static_cast<long long>(k0 + j) * dk + d]);
    }
    if (d < dk) pp[2 + d] = acc;
  }
  if (lane == 0) {
    pp[0] = mx;
    pp[1] = l;
  }
}

// Merge of the chunk partials of one (row, head): lane c holds chunk c's (max, Σp) —
// up to 64 chunks per pass, loaded in parallel — then each lane owns output dims and
// sums the chunks' Σp·v with weights exp(max_c − M) / Σ_c exp(max_c − M)·Σp_c.
template <typename T>
__global__ __launch_bounds__(64) void attn_combine_kernel(AttnArgs a, const int32_t* __restrict__ pos,
                                                          int max_chunks, const float* __restrict__ part) {
  __shared__ float s_w[kCombineMax];
  const int lane = threadIdx.x;
  const int bh = blockIdx.x;
  const int b = bh / a.H, h = bh - (bh / a.H) * a.H;
  const int dk = a.dk, ps = dk + 2;
  const int len = pos[b] + 1;
  const int nc = (len + kTile - 1) / kTile;
  const float* pb = part + static_cast<size_t>(bh) * max_chunks * ps;
  float M = -INFINITY;
  for (int c = lane; c < nc; c += 64) M = fmaxf(M, pb[c * ps]);
  M = wave_max(M);
  float den = 0.f;
  for (int c = lane; c < nc; c += 64) {
    const float w = expf(pb[c * ps] - M);
    s_w[c] = w;
    den += w * pb[c * ps + 1];
  }
  den = wave_sum(den);
  __syncthreads();
  const float inv = 1.f / den;
  T* out = static_cast<T*>(a.out) + static_cast<size_t>(b) * a.H * dk + h * dk;
  for (int d = lane; d < dk; d += 64) {
    float num = 0.f;
    for (int c = 0; c < nc; ++c) num += s_w[c] * pb[c * ps + 2 + d];
    out[d] = static_cast<T>(num * inv);
  }
}

// Causal flash attention on the matrix cores (fp16, head dim 64 or 128) for the calls
// that store the softmax statistics (the backward recomputes the scores from them), so
// the scores are rounded to fp16 as in the scalar path. A 256-lane workgroup takes 128
// queries of one (row, head), 32 per wave, and walks 64-key tiles of the cache staged
// in LDS (K row-major, V transposed):
//   Sᵀ = K·Qᵀ    v_mfma_f32_32x32x16_f16, A = 32 keys × 16 dims from LDS, B = Qᵀ
//                (registers for the whole walk); lane l then holds query l%32 and
//                keys 8(r/4) + 4(l/32) + r%4 of each 32-key tile in register r;
//   online softmax per query: lane-local over its 16 keys, one xor-32 shuffle with
//                the lane holding the other 16;
//   Oᵀ += Vᵀ·Pᵀ  A = Vᵀ (32 dims × 16 keys) from LDS, B = Pᵀ in fp16 straight from the
//                Sᵀ registers: B's k-slot j of lane l is key 8(j/4) + 4(l/32) + j%4 of
//                the 16-key block, and A is read with the same key order;
// so each lane owns one query's output column: the α rescale and the final 1/Σp
// need no data exchange. Key tiles past a wave's last query are skipped; the next
// tile's K/V are loaded into registers while the current one is multiplied; query
// tiles are dispatched last-first (the causal walk is longest for them).
constexpr int kFQ = 128, kFK = 64;

template <int DK>
__global__ __launch_bounds__(256, 2) void attn_prefill_mfma_kernel(AttnArgs a) {
#pragma clang fp contract(off)
  constexpr int KS = DK / 16;  // 16-dim steps of q·k
  constexpr int OT = DK / 32;  // 32-dim tiles of the output
  __shared__ half_t Ks[kFK][DK + 8];
  // Vt rows 34 dwords apart: the 32 rows one ds_read_b64 phase reads (lanes 0-31, and
  // 32-63) fall on 32 distinct bank pairs of the 64 banks (36 dwords put rows r and
  // r + 16 on the same bank: 33 % of LDS cycles were conflicts).
  __shared__ half_t Vt[DK][kFK + 4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // Workgroup n runs on XCD n % 8. Give all query tiles of one (row, head) to one XCD,
  // one after another, so that head's K/V stay in that XCD's L2.
  const int nq = gridDim.x;
  int bh = blockIdx.y, qt = blockIdx.x;
  if (gridDim.y % 8 == 0) {
    const int n = blockIdx.x + blockIdx.y * nq;
    const int slot = n >> 3;
    bh = (n & 7) + 8 * (slot / nq);
    qt = slot % nq;
  }
  const int b = bh / a.H, h = bh - (bh / a.H) * a.H;
  const int S = a.seq_len ? a.seq_len[b] : a.S;
  const int q0 = (nq - 1 - qt) * kFQ;
  if (q0 >= S) return;  // past a ragged sequence's end (uniform over the workgroup)
  const int base = a.pos_base ? a.pos_base[b] : 0;
  const half_t* __restrict__ Kg = static_cast<const half_t*>(a.k) + b * a.kv_stride_b + h * a.kv_stride_h;
  const half_t* __restrict__ Vg = static_cast<const half_t*>(a.v) + b * a.kv_stride_b + h * a.kv_stride_h;
  const half_t* __restrict__ Qg = static_cast<const half_t*>(a.q) + static_cast<size_t>(bh) * a.S * DK;
  const float scale_t = static_cast<float>(static_cast<half_t>(a.scale));
  // rnd(rnd(q·k) / s) for fp16 s = p / 2^e (DK 64: s = 8; DK 128: s = 181/16): the
  // fp32 product with the correctly rounded reciprocal rounds to the same fp16 value —
  // the exact quotient of an fp16 by s is never within 2^-19 (relative) of an fp16
  // rounding midpoint, far beyond the product's 2^-23 error.
  const float rscale = 1.0f / scale_t;
  const int qw = q0 + wave * 32;           // first query of this wave
  const int myq = qw + (lane & 31);        // this lane's query
  const int hi = lane >> 5;                // which half of the wave
  const half8 z8 = {0, 0, 0, 0, 0, 0, 0, 0};
  half8 qb[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks)
    qb[ks] = myq < S ? *reinterpret_cast<const half8*>(Qg + static_cast<size_t>(myq) * DK + ks * 16 + hi * 8)
                     : z8;
  const int kend = base + min(q0 + kFQ, S);  // keys of the workgroup's last query
  const int wave_last = base + min(qw + 31, S - 1);
  const int qpos = base + myq;
  float m = -INFINITY, l = 0.f;
  floatx16 o[OT];
#pragma unroll
  for (int t = 0; t < OT; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[t][r] = 0.f;

  // Per tile each thread holds CH 16-byte pieces of K (key-major) and CH of V. The V
  // pieces come as key pairs (keys 2p, 2p+1 of the same 8 dims, p = tid % 32) so the
  // transposed store is one 4-byte word per dim, 32 lanes covering a contiguous
  // 128-byte row segment of Vt: no bank conflicts.
  constexpr int CH = kFK * DK / 8 / 256;
  constexpr int VG = DK / 8;                  // 8-dim groups of a key
  half8 kn[CH], vn[CH];
  // (keys past kend only in the last tile: the bounds test is made there alone)
  auto fetch_tile = [&](int k0, bool full) {
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const int c = tid + 256 * i;
      const int key = c / VG, d8 = (c % VG) * 8;
      const bool ok = full || k0 + key < kend;
      kn[i] = ok ? *reinterpret_cast<const half8*>(Kg + static_cast<long long>(k0 + key) * DK + d8) : z8;
    }
#pragma unroll
    for (int i = 0; i < CH / 2; ++i) {
      const int grp = (tid >> 5) + 8 * i;     // 8-dim group
      const int key = 2 * (tid & 31);
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const bool ok = full || k0 + key + u < kend;
        vn[2 * i + u] = ok ? *reinterpret_cast<const half8*>(Vg + static_cast<long long>(k0 + key + u) * DK + grp * 8)
                           : z8;
      }
    }
  };
  auto fetch = [&](int k0) {
    if (k0 + kFK <= kend)
      fetch_tile(k0, true);
    else
      fetch_tile(k0, false);
  };
  fetch(0);
  for (int k0 = 0; k0 < kend; k0 += kFK) {
    __syncthreads();
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const int c = tid + 256 * i;
      const int key = c / VG, d8 = (c % VG) * 8;
      *reinterpret_cast<half8*>(&Ks[key][d8]) = kn[i];
    }
#pragma unroll
    for (int i = 0; i < CH / 2; ++i) {
      const int grp = (tid >> 5) + 8 * i, key = 2 * (tid & 31);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        typedef _Float16 half2v __attribute__((ext_vector_type(2)));
        const half2v pr = {vn[2 * i][e], vn[2 * i + 1][e]};
        *reinterpret_cast<half2v*>(&Vt[grp * 8 + e][key]) = pr;
      }
    }
    __syncthreads();
    if (k0 + kFK < kend) fetch(k0 + kFK);
    if (k0 > wave_last) continue;  // every key of this tile is after this wave's queries
    floatx16 st[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
#pragma unroll
      for (int r = 0; r < 16; ++r) st[t][r] = 0.f;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const half8 ka = *reinterpret_cast<const half8*>(&Ks[t * 32 + (lane & 31)][ks * 16 + hi * 8]);
        st[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka, qb[ks], st[t], 0, 0, 0);
      }
    }
    {
      // Scores as fp16 pairs (registers r = 2c, 2c + 1): rnd(rnd(q·k)·rscale) is one mixed
      // fma with an fp16 result (the exact product rounds as its fp32 rounding does, see
      // rscale), the running maximum a packed fp16 max.
      typedef _Float16 half2v __attribute__((ext_vector_type(2)));
      half2v sp[2][8];
      half2v mp = {static_cast<_Float16>(-INFINITY), static_cast<_Float16>(-INFINITY)};
      auto score = [&](float acc) {
        return static_cast<_Float16>(__builtin_fmaf(static_cast<float>(static_cast<_Float16>(acc)), rscale, 0.f));
      };
      if (k0 + kFK - 1 > base + qw) {  // the tile reaches past some query of this wave: mask
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int c = 0; c < 8; ++c) {
            half2v v;
#pragma unroll
            for (int u = 0; u < 2; ++u) {
              const int r = 2 * c + u;
              const int key = k0 + t * 32 + 8 * (r >> 2) + 4 * hi + (r & 3);
              v[u] = (key <= qpos && key < kend) ? score(st[t][r]) : static_cast<_Float16>(-INFINITY);
            }
            sp[t][c] = v;
            mp = __builtin_elementwise_max(mp, v);
          }
      } else {  // every key of the tile precedes every query of the wave
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int c = 0; c < 8; ++c) {
            const half2v v = {score(st[t][2 * c]), score(st[t][2 * c + 1])};
            sp[t][c] = v;
            mp = __builtin_elementwise_max(mp, v);
          }
      }
      float mx = fmaxf(m, fmaxf(static_cast<float>(mp[0]), static_cast<float>(mp[1])));
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      constexpr float kLog2e = 1.4426950408889634f;
      const float alpha = (mx == -INFINITY) ? 1.f : __builtin_amdgcn_exp2f((m - mx) * kLog2e);
      const float nmx = -mx * kLog2e;  // exp(s - mx) as exp2(s·log2 e − mx·log2 e), one FMA a score
      l *= alpha;
      // alpha is exactly 1 where the running max did not grow; the accumulators are
      // rescaled only when some lane's max grew (rare after the first tiles)
      if (__any(mx > m)) {
#pragma unroll
        for (int t = 0; t < OT; ++t)
#pragma unroll
          for (int r = 0; r < 16; ++r) o[t][r] *= alpha;
      }
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
          half8 pb;
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            // mx is finite (key 0 precedes every query, and tiles run from key 0), so a
            // masked score gives exp2(-inf) = 0
            const float sv = static_cast<float>(sp[t][(8 * kb + j) >> 1][j & 1]);
            const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(sv, kLog2e, nmx));
            l += p;
            pb[j] = static_cast<half_t>(p);
          }
          const int kblk = t * 32 + kb * 16 + 4 * hi;
#pragma unroll
          for (int ot = 0; ot < OT; ++ot) {
            const half_t* vrow = &Vt[ot * 32 + (lane & 31)][kblk];
            half8 va;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              va[e] = vrow[e];
              va[4 + e] = vrow[8 + e];
            }
            o[ot] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, pb, o[ot], 0, 0, 0);
          }
        }
      m = mx;
    }
  }
  l += __shfl_xor(l, 32, 64);
  if (myq < S && a.lse && hi == 0) a.lse[static_cast<size_t>(bh) * a.S + myq] = m + logf(l);
  if (myq < S && a.m_out && hi == 0) {
    a.m_out[static_cast<size_t>(bh) * a.S + myq] = m;
    a.l_out[static_cast<size_t>(bh) * a.S + myq] = l;
  }
  if (myq < S) {
    const float inv = 1.f / l;
    const int hd = a.H * DK;
    const size_t row = (a.row_start ? a.row_start[b] : static_cast<size_t>(b) * S) + myq;
    half_t* out = static_cast<half_t*>(a.out) + row * hd + h * DK;
#pragma unroll
    for (int ot = 0; ot < OT; ++ot)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        out[ot * 32 + 8 * (r >> 2) + 4 * hi + (r & 3)] = static_cast<half_t>(o[ot][r] * inv);
  }
}

// Causal flash attention on the matrix cores with fp32 scores (prefill calls that keep
// no softmax statistics), software-pipelined over the 64-key tiles. The layout per wave
// is attn_prefill_mfma_kernel's (32 queries, Sᵀ = K·Qᵀ and Oᵀ += Vᵀ·Pᵀ on
// v_mfma_f32_32x32x16_f16, each lane owning one query's softmax state and output
// column); what differs is the order of the work. Iteration j of a wave:
//   1. one barrier; K of tile j + 2 and V of tile j + 1 go from registers into LDS (two
//      buffers each: K(j + 2) replaces K(j), read one iteration earlier; V(j + 1)
//      replaces V(j − 1)), and the loads of K(j + 3) and V(j + 2) are issued;
//   2. the rescale of O and l when tile j moved a query's reference point (rare: the
//      point moves only when a maximum grows by more than 2^8 in p);
//   3. the scores of tile j + 1 (16 MFMAs) beside the probabilities of tile j (exp2,
//      fp16 packing, row sums) — independent work for the matrix and vector pipes;
//   4. P·V of tile j (16 MFMAs) beside the masking, maximum and reference point of
//      tile j + 1.
// Rows past the last key are read clamped to it (in bounds and finite; the causal
// mask removes them), so a tile needs no bounds tests. Waves whose queries all lie
// past the sequence skip the arithmetic but join the barriers.
template <int DK>
__global__ __launch_bounds__(256, 2) void attn_prefill_pipe_kernel(AttnArgs a) {
#pragma clang fp contract(off)
  constexpr int KS = DK / 16;  // 16-dim steps of q·k
  constexpr int OT = DK / 32;  // 32-dim tiles of the output
  constexpr int CH = kFK * DK / 8 / 256;  // 16-byte pieces of a tile's K (and of V) per thread
  constexpr int VG = DK / 8;              // 8-dim groups of a key
  __shared__ half_t Ks[2][kFK][DK + 8];
  __shared__ half_t Vt[2][DK][kFK + 4];  // rows 34 dwords apart, as in attn_prefill_mfma_kernel
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nq = gridDim.x;
  int bh = blockIdx.y, qt = blockIdx.x;
  if (gridDim.y % 8 == 0) {  // all query tiles of one (row, head) on one XCD
    const int n = blockIdx.x + blockIdx.y * nq;
    const int slot = n >> 3;
    bh = (n & 7) + 8 * (slot / nq);
    qt = slot % nq;
  }
  const int b = bh / a.H, h = bh - (bh / a.H) * a.H;
  const int S = a.seq_len ? a.seq_len[b] : a.S;
  const int q0 = (nq - 1 - qt) * kFQ;
  if (q0 >= S) return;  // past a ragged sequence's end (uniform over the workgroup)
  const int base = a.pos_base ? a.pos_base[b] : 0;
  const half_t* __restrict__ Kg = static_cast<const half_t*>(a.k) + b * a.kv_stride_b + h * a.kv_stride_h;
  const half_t* __restrict__ Vg = static_cast<const half_t*>(a.v) + b * a.kv_stride_b + h * a.kv_stride_h;
  const half_t* __restrict__ Qg = static_cast<const half_t*>(a.q) + static_cast<size_t>(bh) * a.S * DK;
  const float scale_t = static_cast<float>(static_cast<half_t>(a.scale));
  const float cscale = 1.4426950408889634f / scale_t;  // log2(e) / scale
  const float lazy = 8.0f / cscale;                     // 2^8 in p, in units of q·k
  const int qw = q0 + wave * 32;     // first query of this wave
  const int myq = qw + (lane & 31);  // this lane's query
  const int hi = lane >> 5;          // which half of the wave
  const int qpos = base + myq;
  const half8 z8 = {0, 0, 0, 0, 0, 0, 0, 0};
  half8 qb[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks)
    qb[ks] = myq < S ? *reinterpret_cast<const half8*>(Qg + static_cast<size_t>(myq) * DK + ks * 16 + hi * 8)
                     : z8;
  const int kend = base + min(q0 + kFQ, S);  // keys of the workgroup's last query
  const int nt = (kend + kFK - 1) / kFK;     // key tiles of the workgroup
  const int ntw = qw < S ? (base + min(qw + 31, S - 1)) / kFK + 1 : 0;  // tiles this wave reads

  // K and V through buffer loads: bytes past the last key (kend rows) read as zero, so
  // a tile needs no bounds tests (the causal mask removes those keys), and a tile's
  // offset is a scalar added to a fixed per-thread offset.
  const int kv_bytes = kend * DK * static_cast<int>(sizeof(half_t));
  const __amdgpu_buffer_rsrc_t kres =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<half_t*>(Kg), static_cast<short>(0), kv_bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t vres =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<half_t*>(Vg), static_cast<short>(0), kv_bytes, 0x00020000);
  constexpr int kTileBytes = kFK * DK * 2;
  const int koff = (tid / VG) * DK * 2 + (tid % VG) * 16;  // piece i: + i·4096 bytes (256/VG keys)
  const int voff = 2 * (tid & 31) * DK * 2 + (tid >> 5) * 16;
  half8 kn[CH], vn[CH];
  auto fetch_k = [&](int t, half8 (&dst)[CH]) {
#pragma unroll
    for (int i = 0; i < CH; ++i)
      dst[i] = __builtin_bit_cast(half8, __builtin_amdgcn_raw_buffer_load_b128(kres, koff, t * kTileBytes + i * 4096, 0));
  };
  // V as key pairs (keys 2p, 2p + 1 of the same 8 dims, p = tid % 32): the transposed
  // store is one 4-byte word per dim, 32 lanes covering a 128-byte row segment of Vt
  auto fetch_v = [&](int t) {
#pragma unroll
    for (int i = 0; i < CH / 2; ++i)
#pragma unroll
      for (int u = 0; u < 2; ++u)
        vn[2 * i + u] = __builtin_bit_cast(
            half8, __builtin_amdgcn_raw_buffer_load_b128(vres, voff + u * DK * 2 + i * 128, t * kTileBytes, 0));
  };
  auto put_k = [&](auto buf_c, const half8 (&src)[CH]) {
    constexpr int buf = decltype(buf_c)::value;
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const int c = tid + 256 * i;
      *reinterpret_cast<half8*>(&Ks[buf][c / VG][(c % VG) * 8]) = src[i];
    }
  };
  typedef _Float16 half2v __attribute__((ext_vector_type(2)));
  auto put_v = [&](auto buf_c) {
    constexpr int buf = decltype(buf_c)::value;
#pragma unroll
    for (int i = 0; i < CH / 2; ++i) {
      const int grp = (tid >> 5) + 8 * i, key = 2 * (tid & 31);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const half2v pr = {vn[2 * i][e], vn[2 * i + 1][e]};
        *reinterpret_cast<half2v*>(&Vt[buf][grp * 8 + e][key]) = pr;
      }
    }
  };
  // Sᵀ of one tile: lane l holds query l % 32 and keys 8(r/4) + 4(l/32) + r % 4 of each
  // 32-key half t in register r of s[t]
  auto scores = [&](auto buf_c, floatx16 (&s)[2]) {
    constexpr int buf = decltype(buf_c)::value;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
#pragma unroll
      for (int r = 0; r < 16; ++r) s[t][r] = 0.f;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const half8 ka = *reinterpret_cast<const half8*>(&Ks[buf][t * 32 + (lane & 31)][ks * 16 + hi * 8]);
        s[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka, qb[ks], s[t], 0, 0, 0);
      }
    }
  };

  float m = -INFINITY, l = 0.f;  // reference point (units of q·k) and Σ p of this lane's query
  float mnew = -INFINITY;        // the reference point tile j's probabilities use
  bool grow = false;             // whether it moved (wave-uniform)
  floatx16 o[OT];
#pragma unroll
  for (int t = 0; t < OT; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[t][r] = 0.f;

  // Masking of tile t's scores (keys after the query: −∞), their maximum, and the
  // reference point the tile's probabilities will use. A key tile past the sequence's
  // last key never reaches here (kend bounds the tiles), and key 0 precedes every
  // query, so the reference point is finite from the first tile on.
  auto prep = [&](auto mask_c, int t, floatx16 (&s)[2]) {
    if constexpr (decltype(mask_c)::value) {
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = t * kFK + u * 32 + 8 * (r >> 2) + 4 * hi + (r & 3);
          if (key > qpos) s[u][r] = -INFINITY;
        }
    }
    float mloc = s[0][0];
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        if (u + r > 0) mloc = fmaxf(mloc, s[u][r]);
    float mx = fmaxf(m, mloc);
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    grow = __any(mx > m + lazy);
    mnew = grow ? mx : m;
  };
  auto masked = [&](int t) { return (t + 1) * kFK - 1 > base + qw; };

  // One tile's softmax and P·V, with the next tile's scores (NEXT) beside them. PAR is
  // the tile's parity: its V sits in buffer PAR, the next tile's K in buffer PAR ^ 1
  // (compile-time, so every LDS address is a constant offset from one register).
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using T_ = std::true_type;
  using F_ = std::false_type;
  auto body = [&](auto par_c, auto next_c, auto mask_next_c, int j, floatx16 (&cur)[2], floatx16 (&nxt)[2]) {
    constexpr int PAR = decltype(par_c)::value;
    constexpr bool NEXT = decltype(next_c)::value;
    if (grow) {
      const float alpha = __builtin_amdgcn_exp2f((m - mnew) * cscale);
      l *= alpha;
#pragma unroll
      for (int t = 0; t < OT; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[t][r] *= alpha;
    }
    m = mnew;
    if constexpr (NEXT) scores(std::integral_constant<int, PAR ^ 1>{}, nxt);
    const float nmx = -m * cscale;
    const half2v ones = {static_cast<_Float16>(1.0f), static_cast<_Float16>(1.0f)};
    half8 pb[4];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int jj = 0; jj < 8; jj += 2) {
          const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(cur[t][8 * kb + jj], cscale, nmx));
          const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(cur[t][8 * kb + jj + 1], cscale, nmx));
          const half2v pp = {static_cast<_Float16>(p0), static_cast<_Float16>(p1)};
          l = __builtin_amdgcn_fdot2(pp, ones, l, false);
          pb[2 * t + kb][jj] = pp[0];
          pb[2 * t + kb][jj + 1] = pp[1];
        }
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const int kblk = t * 32 + kb * 16 + 4 * hi;
#pragma unroll
        for (int ot = 0; ot < OT; ++ot) {
          const half_t* vrow = &Vt[PAR][ot * 32 + (lane & 31)][kblk];
          half8 va;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            va[e] = vrow[e];
            va[4 + e] = vrow[8 + e];
          }
          o[ot] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, pb[2 * t + kb], o[ot], 0, 0, 0);
        }
      }
    if constexpr (NEXT) prep(mask_next_c, j + 1, nxt);
  };
  auto iter = [&](auto par_c, int j, floatx16 (&cur)[2], floatx16 (&nxt)[2]) {
    constexpr int PAR = decltype(par_c)::value;
    __syncthreads();
    if (j + 2 < nt) put_k(par_c, kn);
    if (j + 1 < nt) put_v(std::integral_constant<int, PAR ^ 1>{});
    if (j + 3 < nt) fetch_k(j + 3, kn);
    if (j + 2 < nt) fetch_v(j + 2);
    if (j >= ntw) return;
    if (j + 1 >= ntw)
      body(par_c, F_{}, F_{}, j, cur, nxt);
    else if (masked(j + 1))
      body(par_c, T_{}, T_{}, j, cur, nxt);
    else
      body(par_c, T_{}, F_{}, j, cur, nxt);
  };

  floatx16 sA[2], sB[2];
  {  // prologue: K(0), V(0), K(1) into LDS; K(2), V(1) into registers; tile 0's scores
    half8 k1[CH];
    fetch_k(0, kn);
    fetch_v(0);
    if (nt > 1) fetch_k(1, k1);
    put_k(I0{}, kn);
    put_v(I0{});
    if (nt > 1) put_k(I1{}, k1);
    if (nt > 2) fetch_k(2, kn);
    if (nt > 1) fetch_v(1);
    __syncthreads();
    if (ntw > 0) {
      scores(I0{}, sA);
      if (masked(0))
        prep(T_{}, 0, sA);
      else
        prep(F_{}, 0, sA);
    }
  }
  for (int j = 0; j < nt; j += 2) {
    iter(I0{}, j, sA, sB);
    if (j + 1 < nt) iter(I1{}, j + 1, sB, sA);
  }
  l += __shfl_xor(l, 32, 64);
  if (myq < S) {
    const float inv = 1.f / l;
    const int hd = a.H * DK;
    const size_t row = (a.row_start ? a.row_start[b] : static_cast<size_t>(b) * S) + myq;
    half_t* out = static_cast<half_t*>(a.out) + row * hd + h * DK;
#pragma unroll
    for (int ot = 0; ot < OT; ++ot)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        out[ot * 32 + 8 * (r >> 2) + 4 * hi + (r & 3)] = static_cast<half_t>(o[ot][r] * inv);
  }
}


// fp32 causal prefill on MFMA 32×32×2 (head dims 64 and 128): 4 waves × 32 queries per
// block, key tiles of 64 through LDS. Each wave computes Sᵀ = K·Qᵀ (keys as rows) so
// that lane l and lane l ^ 32 own query l % 32: the online-softmax state is per lane,
// and Oᵀ = Vᵀ·Pᵀ takes the probabilities straight from the registers (lane l supplies
// key rows f(r) for k = 0 and f(r) + 4 for k = 1 of the 32 × 32 tile, which only
// reorders the sum). Scores are q·k / scale in fp32 as in attn_prefill_kernel.
constexpr int kF32Q = 128, kF32K = 64;

template <int DK>
constexpr size_t f32_mfma_lds() {
  return 2 * kF32K * (DK + 1) * sizeof(float);
}

template <int DK>
__global__ __launch_bounds__(256) void attn_prefill_f32_mfma(AttnArgs a) {
  extern __shared__ float lds[];
  constexpr int P = DK + 1, NJ = DK / 32;
  float* Ks = lds;
  float* Vs = lds + kF32K * P;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, l32 = lane & 31, hi = lane >> 5;
  const int bh = blockIdx.y, b = bh / a.H, h = bh - (bh / a.H) * a.H;
  const int S = a.seq_len ? a.seq_len[b] : a.S;
  const int q0 = blockIdx.x * kF32Q;
  if (q0 >= S) return;  // past a ragged sequence's end (uniform over the block)
  const int base = a.pos_base ? a.pos_base[b] : 0;
  const int s = q0 + 32 * w + l32;
  const bool valid = s < S;
  const int qpos = base + (valid ? s : S - 1);
  const int kv_end = base + min(S, q0 + kF32Q);                  // keys of the block
  const int wave_last = base + min(S - 1, q0 + 32 * w + 31);     // last key this wave needs
  const float* __restrict__ K = static_cast<const float*>(a.k) + b * a.kv_stride_b + h * a.kv_stride_h;
  const float* __restrict__ V = static_cast<const float*>(a.v) + b * a.kv_stride_b + h * a.kv_stride_h;
  float qr[DK / 2];  // Q[s][2i + hi]: the B operand of Sᵀ
  {
    const float* qp = static_cast<const float*>(a.q) +
                      (static_cast<size_t>(bh) * a.S + (valid ? s : S - 1)) * DK + hi;
#pragma unroll
    for (int i = 0; i < DK / 2; ++i) qr[i] = qp[2 * i];
  }
  floatx16 o[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[j][r] = 0.f;
  float m = -INFINITY, l = 0.f;
  // the next K/V tile is loaded into registers while the current one multiplies
  floatx4 nk[DK / 16], nv[DK / 16];
  auto fetch = [&](int k0) {
#pragma unroll
    for (int i = 0; i < DK / 16; ++i) {
      const int e = threadIdx.x + 256 * i;
      const int r = e / (DK / 4), c = (e - r * (DK / 4)) * 4;
      const floatx4 z = {0.f, 0.f, 0.f, 0.f};
      const bool ok = k0 + r < kv_end;
      nk[i] = ok ? *reinterpret_cast<const floatx4*>(K + static_cast<long long>(k0 + r) * DK + c) : z;
      nv[i] = ok ? *reinterpret_cast<const floatx4*>(V + static_cast<long long>(k0 + r) * DK + c) : z;
    }
  };
  fetch(0);
  for (int k0 = 0; k0 < kv_end; k0 += kF32K) {
    __syncthreads();  // every wave is done with the previous tile
#pragma unroll
    for (int i = 0; i < DK / 16; ++i) {
      const int e = threadIdx.x + 256 * i;
      const int r = e / (DK / 4), c = (e - r * (DK / 4)) * 4;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        Ks[r * P + c + j] = nk[i][j];
        Vs[r * P + c + j] = nv[i][j];
      }
    }
    __syncthreads();
    if (k0 + kF32K < kv_end) fetch(k0 + kF32K);
    if (k0 > wave_last) continue;  // every key of the tile is after this wave's queries
    floatx16 sc[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
#pragma unroll
      for (int r = 0; r < 16; ++r) sc[t][r] = 0.f;
      const float* ka = Ks + (32 * t + l32) * P + hi;
#pragma unroll
      for (int i = 0; i < DK / 2; ++i)
        sc[t] = __builtin_amdgcn_mfma_f32_32x32x2f32(ka[2 * i], qr[i], sc[t], 0, 0, 0);
    }
    float mloc = -INFINITY;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = k0 + 32 * t + 8 * (r >> 2) + 4 * hi + (r & 3);
        const float v = key <= qpos ? sc[t][r] / a.scale : -INFINITY;
        sc[t][r] = v;
        mloc = fmaxf(mloc, v);
      }
    mloc = fmaxf(mloc, __shfl_xor(mloc, 32, 64));
    // finite: the first tile holds key 0, which every query sees
    const float mn = fmaxf(m, mloc);
    const float alpha = expf(m - mn);
    float lsum = 0.f;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = expf(sc[t][r] - mn);
        sc[t][r] = p;
        lsum += p;
      }
    l = l * alpha + (lsum + __shfl_xor(lsum, 32, 64));
    m = mn;
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[j][r] *= alpha;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float* vrow = Vs + (32 * t + 8 * (r >> 2) + 4 * hi + (r & 3)) * P + l32;
#pragma unroll
        for (int j = 0; j < NJ; ++j)
          o[j] = __builtin_amdgcn_mfma_f32_32x32x2f32(vrow[32 * j], sc[t][r], o[j], 0, 0, 0);
      }
  }
  if (valid) {
    const size_t row = (a.row_start ? a.row_start[b] : static_cast<size_t>(b) * a.S) + s;
    float* out = static_cast<float*>(a.out) + row * a.H * DK + h * DK;
    const float inv = 1.f / l;
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) out[32 * j + 8 * (r >> 2) + 4 * hi + (r & 3)] = o[j][r] * inv;
    if (a.lse && hi == 0) a.lse[static_cast<size_t>(bh) * a.S + s] = m + logf(l);
    if (a.m_out && hi == 0) {
      a.m_out[static_cast<size_t>(bh) * a.S + s] = m;
      a.l_out[static_cast<size_t>(bh) * a.S + s] = l;
    }
  }
}

template <int DK>
int prefill_f32_mfma(const AttnArgs& a, hipStream_t st) {
  constexpr size_t lds = f32_mfma_lds<DK>();
  static bool attr = false;
  if (!attr) {
    NML_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(&attn_prefill_f32_mfma<DK>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)));
    attr = true;
  }
  dim3 grid((a.S + kF32Q - 1) / kF32Q, a.B * a.H);
  attn_prefill_f32_mfma<DK><<<grid, 256, lds, st>>>(a);
  NML_LAUNCHED();
  return 0;
}

template <typename T, int DK>
int prefill_typed(const AttnArgs& a, hipStream_t st) {
  if (a.full) {  // non-causal / masked: the scalar kernel only
    NML_REQUIRE(!a.pos_base && !a.seq_len && !a.row_start,
                "attention: non-causal attention takes dense rows from position 0");
    dim3 grid((a.S + kTile - 1) / kTile, a.B * a.H);
    attn_prefill_kernel<T, DK><<<grid, 64, 0, st>>>(a);
    NML_LAUNCHED();
    return 0;
  }
  if constexpr (sizeof(T) == 4 && (DK == 64 || DK == 128)) {
    if (!std::getenv("NIMBLEML_ATTN_F32_SCALAR")) return prefill_f32_mfma<DK>(a, st);
  }
  if constexpr (sizeof(T) == 2 && (DK == 64 || DK == 128)) {
    dim3 grid((a.S + kFQ - 1) / kFQ, a.B * a.H);
    // fp16-rounded scores where the backward recomputes them from the statistics
    // The pipelined kernel's buffer loads take a 32-bit byte range per (row, head): a
    // cache row block past 2 GiB (kv_stride_h elements) takes the other kernel.
    const bool ranged = a.kv_stride_h * static_cast<long long>(sizeof(half_t)) < (1LL << 31);
    if (a.lse || a.m_out || !ranged)
      attn_prefill_mfma_kernel<DK><<<grid, 256, 0, st>>>(a);
    else
      attn_prefill_pipe_kernel<DK><<<grid, 256, 0, st>>>(a);
    NML_LAUNCHED();
    return 0;
  }
  dim3 grid((a.S + kTile - 1) / kTile, a.B * a.H);
  attn_prefill_kernel<T, DK><<<grid, 64, 0, st>>>(a);
  NML_LAUNCHED();
  return 0;
}

template <typename T, int DK>
int decode_group(const AttnArgs& a, const int32_t* pos, int max_len, void* ws, hipStream_t st) {
  constexpr int G = dec_groups<T, DK>();
  const int max_groups = (max_len + kTile * G - 1) / (kTile * G);
  unsigned long long* part = static_cast<unsigned long long*>(ws);
  attn_decode_group_kernel<T, DK, G><<<dim3(max_groups, a.B * a.H), 256, 0, st>>>(
      a, pos, max_groups, part);
  NML_LAUNCHED();
  return 0;
}

template <typename T>
int decode_chunks(const AttnArgs& a, const int32_t* pos, int max_len, void* ws, hipStream_t st) {
  const int max_chunks = (max_len + kTile - 1) / kTile;
  float* part = static_cast<float*>(ws);
  attn_decode_small_kernel<T><<<dim3(max_chunks, a.B * a.H), 64, 0, st>>>(a, pos, max_chunks, part);
  NML_LAUNCHED();
  attn_combine_kernel<T><<<a.B * a.H, 64, 0, st>>>(a, pos, max_chunks, part);
  NML_LAUNCHED();
  return 0;
}

template <typename T, int DPL>
int prefill_quad(const AttnArgs& a, hipStream_t st) {
  dim3 grid((a.S + 63) / 64, a.B * a.H);
  attn_prefill_quad_kernel<T, DPL><<<grid, 256, 0, st>>>(a);
  NML_LAUNCHED();
  return 0;
}

template <typename T>
int prefill_dk(const AttnArgs& a, hipStream_t st) {
  switch (a.dk) {
    case 8: return prefill_typed<T, 8>(a, st);
    case 16: return prefill_typed<T, 16>(a, st);
    case 32: return prefill_typed<T, 32>(a, st);
    case 64: return prefill_typed<T, 64>(a, st);
    case 128: return prefill_typed<T, 128>(a, st);
  }
  // other head dims: four lanes per query, dims padded to 32, 64, 128 or 256
  if (a.dk <= 32) return prefill_quad<T, 8>(a, st);
  if (a.dk <= 64) return prefill_quad<T, 16>(a, st);
  if (a.dk <= 128) return prefill_quad<T, 32>(a, st);
  if (a.dk <= kMaxHeadDim) return prefill_quad<T, 64>(a, st);
  set_error("attention: head_dim %d above %d", a.dk, kMaxHeadDim);
  return -1;
}

template <typename T>
int decode_dk(const AttnArgs& a, const int32_t* pos, int max_len, void* ws, hipStream_t st) {
  switch (a.dk) {
    case 32: return decode_group<T, 32>(a, pos, max_len, ws, st);
    case 64: return decode_group<T, 64>(a, pos, max_len, ws, st);
    case 128: return decode_group<T, 128>(a, pos, max_len, ws, st);
    case 256: return decode_group<T, 256>(a, pos, max_len, ws, st);
  }
  if (a.dk < 1 || a.dk > kMaxHeadDim) {
    set_error("attention: head_dim %d outside [1, %d]", a.dk, kMaxHeadDim);
    return -1;
  }
  return decode_chunks<T>(a, pos, max_len, ws, st);
}

}  // namespace

size_t attention_decode_workspace(int B, int H, int dk, int max_len) {
  // head dims ≥ 32: flagged group partials (at most 4 chunks a group
  // never fewer than 1); below: float chunk partials for the combine pass
  const size_t chunks = (max_len + kTile - 1) / kTile;
  const size_t grouped = static_cast<size_t>(B) * H * chunks * dec_slots(dk) * 8;
  const size_t plain = static_cast<size_t>(B) * H * chunks * (dk + 2) * sizeof(float);
  return grouped > plain ? grouped : plain;
}

int launch_attention_prefill(int dt, const AttnArgs& a, hipStream_t st) {
  if (a.B * a.S == 0) return 0;
  return dt == F16 ? prefill_dk<half_t>(a, st) : prefill_dk<float>(a, st);
}

int launch_attention_decode(int dt, const AttnArgs& a, const int32_t* pos, int max_len, void* ws,
                            hipStream_t st) {
  if (a.B == 0) return 0;
  NML_REQUIRE(max_len > 0 && max_len <= kCombineMax * kTile,
              "attention decode: max_len %d outside (0, %d]", max_len, kCombineMax * kTile);
  return dt == F16 ? decode_dk<half_t>(a, pos, max_len, ws, st)
                   : decode_dk<float>(a, pos, max_len, ws, st);
}

}  // namespace nml
