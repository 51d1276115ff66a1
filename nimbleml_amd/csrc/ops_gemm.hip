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
//  * skinny_f16: 8 < M ≤ 64 rows (batched decode), MFMA 16×16×32 with optional split-K
//    and a fused RMSNorm of x (see its comment).
#include <cstdlib>
#include <mutex>

#include "gemm_big.hpp"
#include "kernels.hpp"

namespace nml {

namespace {

// Stores the output element (m, n) and returns its stored value, given the bias b[n]
// and residual r[m][n] as floats (ignored by the epilogues that do not use them).
template <typename T, int EPI>
__device__ __forceinline__ float epilogue_with(const LinearArgs& a, int m, int n, float acc,
                                               float bias_v, float resid_v) {
  T* out = static_cast<T*>(a.out);
  const size_t idx = static_cast<size_t>(m) * a.N + n;
  if constexpr (EPI == EPI_NONE) {
    out[idx] = static_cast<T>(acc);
    return rnd<T>(acc);
  } else {
    const float lin = rnd<T>(rnd<T>(acc) + bias_v);
    if constexpr (EPI == EPI_BIAS) {
      out[idx] = static_cast<T>(lin);
      return lin;
    } else if constexpr (EPI == EPI_BIAS_GELU) {
      const float v = rnd<T>(gelu_t<T>(lin));
      out[idx] = static_cast<T>(v);
      if (a.pre_out) static_cast<T*>(a.pre_out)[idx] = static_cast<T>(lin);
      return v;
    } else if constexpr (EPI == EPI_BIAS_RESID) {
      const float v = rnd<T>(resid_v + lin);
      out[idx] = static_cast<T>(v);
      return v;
    } else {  // EPI_QKV
      const QKVDst& q = a.qkv;
      const int which = n / q.d;
      const int within = n - which * q.d;
      const int h = within / q.dk, j = within - h * q.dk;
      int b, s;
      if (q.row_seg) {
        const int rs = q.row_seg[m];
        b = rs >> 16;
        s = rs & 0xffff;
      } else {
        b = m / q.S;
        s = m - b * q.S;
      }
      if (which == 0) {
        T* qp = static_cast<T*>(q.q);
        qp[((static_cast<size_t>(b) * q.H + h) * q.S + s) * q.dk + j] = static_cast<T>(lin);
      } else {
        const int pos = (q.pos_base ? q.pos_base[b] : 0) + s;
        T* kv = static_cast<T*>(which == 1 ? q.k : q.v);
        kv[b * q.kv_stride_b + h * q.kv_stride_h + static_cast<long long>(pos) * q.dk + j] =
            static_cast<T>(lin);
      }
      return lin;
    }
  }
}

template <typename T, int EPI>
__device__ __forceinline__ float epilogue(const LinearArgs& a, int m, int n, float acc) {
  float bias_v = 0.f, resid_v = 0.f;
  if constexpr (EPI != EPI_NONE) bias_v = static_cast<float>(static_cast<const T*>(a.bias)[n]);
  if constexpr (EPI == EPI_BIAS_RESID)
    resid_v = static_cast<float>(static_cast<const T*>(a.resid)[static_cast<size_t>(m) * a.N + n]);
  return epilogue_with<T, EPI>(a, m, n, acc, bias_v, resid_v);
}

// Epilogue of one 32×32 MFMA tile, fp16: this lane's 16 accumulators are rows
// mb + 8(r/4) + r%4 of column n (D layout of v_mfma_f32_32x32x16_f16). The residual
// operands are loaded first, all together (addresses clamped in bounds, loads
// unconditional, so no wait is forced between them); bias_v is b[n].
template <int EPI>
__device__ __forceinline__ void epilogue_tile32(const LinearArgs& a, int mb, int n, const floatx16& acc,
                                                float bias_v) {
  const int M = a.M, N = a.N;
  if constexpr (EPI == EPI_QKV) {
    // The head-major scatter of epilogue_with, with the column's destination worked out
    // once per tile and each row's (sequence, position) stepped from the tile's first
    // row instead of divided out per element.
    if (n >= N) return;
    const QKVDst& q = a.qkv;
    const int which = n / q.d, within = n - which * q.d;
    const int h = within / q.dk, j = within - h * q.dk;
    half_t* const dst = static_cast<half_t*>(which == 0 ? q.q : which == 1 ? q.k : q.v);
    int rb[16], rp[16];  // each row's sequence and position
    if (q.row_seg) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = mb + 8 * (r >> 2) + (r & 3);
        const int v = q.row_seg[m < M ? m : M - 1];
        rb[r] = v >> 16;
        rp[r] = v & 0xffff;
      }
    } else {
      int b = mb / q.S, s0 = mb - b * q.S;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        int s = s0 + 8 * (r >> 2) + (r & 3), bb = b;
        while (s >= q.S) {  // rows past the tile's first sequence (once at most for S ≥ 32)
          s -= q.S;
          ++bb;
        }
        rb[r] = bb;
        rp[r] = s;
      }
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int m = mb + 8 * (r >> 2) + (r & 3);
      if (m >= M) continue;
      const int b = rb[r], s = rp[r];
      const float lin = rnd<half_t>(rnd<half_t>(acc[r]) + bias_v);
      if (which == 0) {
        dst[((static_cast<size_t>(b) * q.H + h) * q.S + s) * q.dk + j] = static_cast<half_t>(lin);
      } else {
        const int pos = (q.pos_base ? q.pos_base[b] : 0) + s;
        dst[b * q.kv_stride_b + h * q.kv_stride_h + static_cast<long long>(pos) * q.dk + j] =
            static_cast<half_t>(lin);
      }
    }
    return;
  }
  float res[16];
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    res[r] = 0.f;
    if constexpr (EPI == EPI_BIAS_RESID) {
      const int m = mb + 8 * (r >> 2) + (r & 3);
      const size_t mc = m < M ? m : M - 1;
      res[r] = static_cast<float>(static_cast<const half_t*>(a.resid)[mc * N + (n < N ? n : N - 1)]);
    }
  }
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int m = mb + 8 * (r >> 2) + (r & 3);
    if (m < M && n < N) epilogue_with<half_t, EPI>(a, m, n, acc[r], bias_v, res[r]);
  }
}

template <int EPI>
__device__ __forceinline__ float bias_at(const LinearArgs& a, int n) {
  if constexpr (EPI == EPI_NONE) return 0.f;
  return static_cast<float>(static_cast<const half_t*>(a.bias)[n < a.N ? n : a.N - 1]);
}

typedef _Float16 half4v __attribute__((ext_vector_type(4)));

// Epilogue of the big GEMM's block tile, fp16, from transposed accumulators
// (big::mainloop with TR: lane l holds row 32i + l%32 of its wave's block and, in
// accumulator r = 4g + q of tile (i, j), column 32j + 8g + 4(l/32) + q). Each wave rounds
// its (TM/2) × (TN/4) block to fp16 — the first rounding of every epilogue, so nothing is
// lost — into its own region of the LDS the main loop no longer needs, as 8-byte runs,
// then reads the region back as runs of 8 consecutive columns of one row and finishes
// each run with epilogue_with's arithmetic: the residual and bias loads and the output
// stores are 16-byte vectors, 8 rows × 128 bytes per wave instruction, instead of 2-byte
// elements. Widths that are not a multiple of 8 (or operands not 16-byte aligned) take
// the same path element by element.
// fp16 tanh by table for the 256 × 256 GELU epilogue: entry i is rnd(tanh_h(t)) for the
// fp16 t of magnitude code kTanhLo + i, so a lookup equals the computed form bit for bit.
// Below the range rnd(tanh t) = t (tanh t = t·(1 − t²/3 + …) and t²/3 < 2^-12, less than
// half an fp16 ulp below t); from code 0x4500 (|t| = 5) on, rnd(tanh t) = 1, the last
// entry's value (1 − tanh t < 2^-12), so indices clamp there (inf included; a NaN t comes
// only from a NaN x, whose GELU is NaN whatever tanh returns). 16 KiB, copied into LDS
// past the epilogue's staging region.
constexpr int kTanhLo = 0x2500, kTanhN = 0x2000;
constexpr size_t kTanhBytes = kTanhN * sizeof(half_t);
__device__ half_t g_tanh_tab[kTanhN];

__global__ __launch_bounds__(256) void tanh_tab_kernel() {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= kTanhN) return;
  const unsigned short code = static_cast<unsigned short>(kTanhLo + i);
  const float t = static_cast<float>(__builtin_bit_cast(half_t, code));
  g_tanh_tab[i] = static_cast<half_t>(tanh_h(t));
}

// Fills g_tanh_tab on the current device before its first use (once per device; the
// first call waits for the fill on `st`, so it cannot be made under stream capture).
int ensure_tanh_tab(hipStream_t st) {
  static std::mutex mu;
  static bool ready[64] = {};
  int dev = 0;
  NML_HIP(hipGetDevice(&dev));
  NML_REQUIRE(dev >= 0 && dev < 64, "device ordinal %d out of range", dev);
  std::lock_guard<std::mutex> lock(mu);
  if (!ready[dev]) {
    tanh_tab_kernel<<<kTanhN / 256, 256, 0, st>>>();
    NML_LAUNCHED();
    NML_HIP(hipStreamSynchronize(st));
    ready[dev] = true;
  }
  return 0;
}

// gelu8_f16 with its tanh looked up in the LDS copy of g_tanh_tab (byte address tab).
__device__ __forceinline__ half8 gelu8_f16_tab(half8 x, const half_t* tab) {
#pragma clang fp contract(off)
  const half_t k = static_cast<half_t>(0.7978845608028654f);
  const half_t c = static_cast<half_t>(0.044715f);
  half8 t = x * c;
  t = t * x;
  t = t * x;
  t = x + t;
  t = t * k;
  typedef unsigned short u16x8 __attribute__((ext_vector_type(8)));
  const u16x8 tb = __builtin_bit_cast(u16x8, t);
  const u16x8 ab = tb & static_cast<unsigned short>(0x7fff);
  const u16x8 sg = tb & static_cast<unsigned short>(0x8000);
  const unsigned short* tabu = reinterpret_cast<const unsigned short*>(tab);
  unsigned int v[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = tabu[min(max(static_cast<int>(ab[e]) - kTanhLo, 0), kTanhN - 1)];
  // all eight reads issued, and complete here, on every lane (in range by the clamp): the
  // selects below stay selects instead of branches around single reads
  asm volatile("" : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]), "+v"(v[4]), "+v"(v[5]),
               "+v"(v[6]), "+v"(v[7]));
  u16x8 r;
#pragma unroll
  for (int e = 0; e < 8; ++e)
    r[e] = ab[e] < kTanhLo ? tb[e] : static_cast<unsigned short>(v[e] | sg[e]);
  const half8 tu = __builtin_bit_cast(half8, r);
  const half8 a = x * static_cast<half_t>(0.5f);
  const half8 bb = tu + static_cast<half_t>(1.0f);
  return a * bb;
}

template <int TM, int TN>
struct Staged {
  static constexpr int R = TM / 2, C = TN / 4, P = C + 8;  // region rows, columns, pitch
  static constexpr size_t Lds = static_cast<size_t>(8) * R * P * sizeof(half_t);
};

// TAB: the GELU's tanh from the LDS table at tanh_tab. NT: 16-byte stores non-temporal
// (outputs of the 256 × 256 tiles, too large to stay in the caches for their consumer,
// are streamed past L2 instead of evicting the operand lines the other tiles still read).
template <int EPI, bool TAB = false, bool NT = false>
__device__ __forceinline__ void epilogue_run8(const LinearArgs& a, int m, int n, half8 h, bool vec,
                                              const half_t* tanh_tab = nullptr) {
  const int N = a.N;
  if constexpr (EPI == EPI_QKV) {
    const QKVDst& q = a.qkv;
    if (q.dk & 7) {  // a run of 8 may cross a head: element by element
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (n + e < N)
          epilogue_with<half_t, EPI_QKV>(a, m, n + e, static_cast<float>(h[e]),
                                         static_cast<float>(static_cast<const half_t*>(a.bias)[n + e]), 0.f);
      return;
    }
    int b, s;
    if (q.row_seg) {
      const int rs = q.row_seg[m];
      b = rs >> 16;
      s = rs & 0xffff;
    } else {
      b = m / q.S;
      s = m - b * q.S;
    }
    const int which = n / q.d, within = n - which * q.d;
    const int hd = within / q.dk, j = within - hd * q.dk;
    half_t* dst = which == 0
        ? static_cast<half_t*>(q.q) + ((static_cast<size_t>(b) * q.H + hd) * q.S + s) * q.dk + j
        : static_cast<half_t*>(which == 1 ? q.k : q.v) + b * q.kv_stride_b + hd * q.kv_stride_h +
              static_cast<long long>((q.pos_base ? q.pos_base[b] : 0) + s) * q.dk + j;
    const half_t* bias = static_cast<const half_t*>(a.bias) + n;
    half8 bv;
    if (vec) {
      bv = *reinterpret_cast<const half8*>(bias);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) bv[e] = bias[e];  // dk % 8 == 0: a run stays inside one head
    }
    const half8 o = h + bv;  // fp16 adds round as rnd(float + float) does
    if (vec) {
      if constexpr (NT)
        __builtin_nontemporal_store(o, reinterpret_cast<half8*>(dst));
      else
        *reinterpret_cast<half8*>(dst) = o;
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) dst[e] = o[e];
    }
    return;
  }
  const size_t row = static_cast<size_t>(m) * N;
  half_t* out = static_cast<half_t*>(a.out) + row;
  half8 bv = {0, 0, 0, 0, 0, 0, 0, 0}, rv = bv;
  if (vec) {
    if constexpr (EPI != EPI_NONE) bv = *reinterpret_cast<const half8*>(static_cast<const half_t*>(a.bias) + n);
    if constexpr (EPI == EPI_BIAS_RESID)
      rv = *reinterpret_cast<const half8*>(static_cast<const half_t*>(a.resid) + row + n);
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e)
      if (n + e < N) {
        if constexpr (EPI != EPI_NONE) bv[e] = static_cast<const half_t*>(a.bias)[n + e];
        if constexpr (EPI == EPI_BIAS_RESID) rv[e] = static_cast<const half_t*>(a.resid)[row + n + e];
      }
  }
  // fp16 arithmetic on the 8 values at once (an fp16 sum rounds as rnd(float + float)
  // does): lin = rnd(rnd(acc) + b), then the epilogue's own op
  half8 o = h, p = h;
  if constexpr (EPI != EPI_NONE) {
    p = h + bv;
    if constexpr (EPI == EPI_BIAS) o = p;
    else if constexpr (EPI == EPI_BIAS_GELU) {
      if constexpr (TAB)
        o = gelu8_f16_tab(p, tanh_tab);
      else
        o = gelu8_f16(p);
    }
    else o = rv + p;  // EPI_BIAS_RESID
  }
  half_t* pre = EPI == EPI_BIAS_GELU && a.pre_out ? static_cast<half_t*>(a.pre_out) + row : nullptr;
  if (vec) {
    if constexpr (NT)
      __builtin_nontemporal_store(o, reinterpret_cast<half8*>(out + n));
    else
      *reinterpret_cast<half8*>(out + n) = o;
    if (pre) *reinterpret_cast<half8*>(pre + n) = p;
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e)
      if (n + e < N) {
        out[n + e] = o[e];
        if (pre) pre[n + e] = p[e];
      }
  }
}

// epilogue_run8's 16-byte case with its bias and residual runs already in registers.
template <int EPI, bool TAB, bool NT>
__device__ __forceinline__ void epilogue_vec8(const LinearArgs& a, int m, int n, half8 h, half8 bv, half8 rv,
                                              const half_t* tanh_tab) {
  const size_t row = static_cast<size_t>(m) * a.N;
  half8 o = h, p = h;
  if constexpr (EPI != EPI_NONE) {
    p = h + bv;
    if constexpr (EPI == EPI_BIAS) {
      o = p;
    } else if constexpr (EPI == EPI_BIAS_GELU) {
      if constexpr (TAB)
        o = gelu8_f16_tab(p, tanh_tab);
      else
        o = gelu8_f16(p);
    } else {
      o = rv + p;  // EPI_BIAS_RESID
    }
  }
  half_t* out = static_cast<half_t*>(a.out) + row + n;
  if constexpr (NT)
    __builtin_nontemporal_store(o, reinterpret_cast<half8*>(out));
  else
    *reinterpret_cast<half8*>(out) = o;
  if constexpr (EPI == EPI_BIAS_GELU)
    if (a.pre_out) *reinterpret_cast<half8*>(static_cast<half_t*>(a.pre_out) + row + n) = p;
}

template <int EPI, int TM, int TN>
__device__ __forceinline__ void epilogue_staged(const LinearArgs& a, int m0, int n0,
                                                const floatx16 (&acc)[TM / 64][TN / 128],
                                                char* lds_raw) {
  typedef Staged<TM, TN> St;
  constexpr int IA = TM / 64, JB = TN / 128, R = St::R, C = St::C, P = St::P;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
  const int wm = wave >> 2, wn = wave & 3;
  half_t* reg = reinterpret_cast<half_t*>(lds_raw) + wave * R * P;
  __syncthreads();  // every wave is done with the main loop's stages
#pragma unroll
  for (int i = 0; i < IA; ++i)
#pragma unroll
    for (int j = 0; j < JB; ++j)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        half4v v;
#pragma unroll
        for (int q = 0; q < 4; ++q) v[q] = static_cast<half_t>(acc[i][j][4 * g + q]);
        *reinterpret_cast<half4v*>(reg + (32 * i + (lane & 31)) * P + 32 * j + 8 * g + 4 * (lane >> 5)) = v;
      }
  // (the wave reads back only its own region: its LDS operations complete in order)
  const int M = a.M, N = a.N;
  uintptr_t ptrs = reinterpret_cast<uintptr_t>(a.out) | reinterpret_cast<uintptr_t>(a.bias) |
                   reinterpret_cast<uintptr_t>(a.resid) | reinterpret_cast<uintptr_t>(a.pre_out);
  if constexpr (EPI == EPI_QKV)
    ptrs |= reinterpret_cast<uintptr_t>(a.qkv.q) | reinterpret_cast<uintptr_t>(a.qkv.k) |
            reinterpret_cast<uintptr_t>(a.qkv.v);
  const bool aligned = (ptrs & 15) == 0;
  const bool vec8 = (N & 7) == 0 && aligned;
  constexpr int CH = C / 8;              // 16-byte runs per region row
  constexpr int IT = R * CH / 64;        // runs per lane
  // 256 × 256 GELU tiles: the tanh table sits right past the staging region
  constexpr bool kGeluTab = EPI == EPI_BIAS_GELU && TM == 256;
  const half_t* tab = reinterpret_cast<const half_t*>(lds_raw + Staged<TM, TN>::Lds);
  if constexpr (EPI == EPI_QKV) if ((a.qkv.dk & 7) == 0) {
    // A lane's runs all sit in one column (the 64 lanes cover whole region rows), so the
    // column's destination (q / k / v, head, lane within the head) is resolved once, and
    // the row's (sequence, position) is stepped from run to run instead of divided. With
    // dk a multiple of 8 (so is d = H·dk) a run of 8 columns stays inside one head.
    static_assert(64 % CH == 0, "runs of a lane share a column");
    constexpr int RS = 64 / CH;  // region rows between a lane's runs
    const QKVDst& q = a.qkv;
    const int c8 = lane % CH, n = n0 + wn * C + c8 * 8;
    const int which = n / q.d, within = n - which * q.d;
    const int hd = within / q.dk, j = within - hd * q.dk;
    half_t* dst0 = static_cast<half_t*>(which == 0 ? q.q : which == 1 ? q.k : q.v);
    half8 bv = {0, 0, 0, 0, 0, 0, 0, 0};
    const bool vec = vec8 && n + 7 < N;
    if (n < N) {
      if (vec) {
        bv = *reinterpret_cast<const half8*>(static_cast<const half_t*>(a.bias) + n);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e)
          if (n + e < N) bv[e] = static_cast<const half_t*>(a.bias)[n + e];
      }
    }
    const int mfirst = m0 + wm * R + lane / CH;
    int b = 0, sq = 0;
    if (!q.row_seg) {
      b = mfirst / q.S;
      sq = mfirst - b * q.S;
    }
#pragma unroll
    for (int it = 0; it < IT; ++it) {
      const int row = lane / CH + it * RS, m = mfirst + it * RS;
      if (it > 0 && !q.row_seg) {
        sq += RS;
        while (sq >= q.S) {
          sq -= q.S;
          ++b;
        }
      }
      if (m >= M || n >= N) continue;
      int bb = b, ss = sq;
      if (q.row_seg) {
        const int rs = q.row_seg[m];
        bb = rs >> 16;
        ss = rs & 0xffff;
      }
      half_t* dst = which == 0
          ? dst0 + ((static_cast<size_t>(bb) * q.H + hd) * q.S + ss) * q.dk + j
          : dst0 + bb * q.kv_stride_b + hd * q.kv_stride_h +
                static_cast<long long>((q.pos_base ? q.pos_base[bb] : 0) + ss) * q.dk + j;
      const half8 o = *reinterpret_cast<const half8*>(reg + row * P + c8 * 8) + bv;
      if (vec) {
        if constexpr (TM == 256)  // non-temporal, as epilogue_run8's NT
          __builtin_nontemporal_store(o, reinterpret_cast<half8*>(dst));
        else
          *reinterpret_cast<half8*>(dst) = o;
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e)
          if (n + e < N) dst[e] = o[e];
      }
    }
    return;
  }
  if constexpr (EPI != EPI_QKV) {
    // A lane's runs share one column (lane % CH): its bias is loaded once and its rows'
    // residual runs all before the first store, so the loads' latencies overlap instead of
    // each run waiting for its own (the residual may be the output itself: every run reads
    // its elements before any is written). Rows past M read row M − 1 and store nothing.
    static_assert(64 % CH == 0, "runs of a lane share a column");
    constexpr int RS = 64 / CH;
    const int c8 = lane % CH, n = n0 + wn * C + c8 * 8;
    if (vec8 && n + 7 < N) {
      const half8 z = {0, 0, 0, 0, 0, 0, 0, 0};
      half8 bv = z, rv[IT];
      if constexpr (EPI != EPI_NONE) bv = *reinterpret_cast<const half8*>(static_cast<const half_t*>(a.bias) + n);
      const int mfirst = m0 + wm * R + lane / CH;
#pragma unroll
      for (int it = 0; it < IT; ++it) {
        rv[it] = z;
        if constexpr (EPI == EPI_BIAS_RESID) {
          const int mc = min(mfirst + it * RS, M - 1);
          rv[it] = *reinterpret_cast<const half8*>(static_cast<const half_t*>(a.resid) +
                                                   static_cast<size_t>(mc) * N + n);
        }
      }
#pragma unroll
      for (int it = 0; it < IT; ++it) {
        const int m = mfirst + it * RS;
        if (m >= M) continue;
        const half8 h = *reinterpret_cast<const half8*>(reg + (lane / CH + it * RS) * P + c8 * 8);
        epilogue_vec8<EPI, kGeluTab, TM == 256>(a, m, n, h, bv, rv[it], tab);
      }
      return;
    }
  }
#pragma unroll
  for (int it = 0; it < IT; ++it) {
    const int id = it * 64 + lane, row = id / CH, c8 = id - row * CH;
    const int m = m0 + wm * R + row, n = n0 + wn * C + c8 * 8;
    const half8 h = *reinterpret_cast<const half8*>(reg + row * P + c8 * 8);
    if (m < M && n < N) epilogue_run8<EPI, kGeluTab, TM == 256>(a, m, n, h, vec8 && n + 7 < N, tab);
  }
}

// EPI_CE epilogue (tied head fused with cross-entropy): the tile's fp16 logits stay in
// the accumulators. From the transposed layout (lane l: row 32i + l%32 of its wave's
// TM/2 × TN/4 block, columns 32j + 8g + 4(l/32) + q), each row's maximum over the
// tile's TN columns is formed from the 2 lanes holding it and the 4 waves along N (LDS),
// then Σ rnd(exp(rnd(x − max))) — ce_rows_kernel's terms, shifted by the tile maximum —
// likewise; the label's logit is written by the lane holding it. Columns past N count
// as −∞ (each tile holds at least one column below N, so the maximum is finite).
template <int TM, int TN>
__device__ __forceinline__ void epilogue_ce(const LinearArgs& a, int m0, int n0,
                                            const floatx16 (&acc)[TM / 64][TN / 128],
                                            char* lds_raw) {
#pragma clang fp contract(off)
  constexpr int IA = TM / 64, JB = TN / 128, R = TM / 2, C = TN / 4;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
  const int wm = wave >> 2, wn = wave & 3, h = lane >> 5, rl = lane & 31;
  const int N = a.N, cb = n0 + wn * C;  // first column of this wave's block
  float* s_max = reinterpret_cast<float*>(lds_raw);  // [2][4][R]
  float* s_sum = s_max + 8 * R;                      // [2][4][R]
  auto logit = [&](int i, int j, int g, int q) {
    const int col = cb + 32 * j + 8 * g + 4 * h + q;
    return col < N ? rnd<half_t>(acc[i][j][4 * g + q]) : -INFINITY;
  };
  __syncthreads();  // every wave is done with the main loop's stages
#pragma unroll
  for (int i = 0; i < IA; ++i) {
    float m = -INFINITY;
#pragma unroll
    for (int j = 0; j < JB; ++j)
#pragma unroll
      for (int g = 0; g < 4; ++g)
#pragma unroll
        for (int q = 0; q < 4; ++q) m = fmaxf(m, logit(i, j, g, q));
    m = fmaxf(m, __shfl_xor(m, 32, 64));
    if (h == 0) s_max[(wm * 4 + wn) * R + 32 * i + rl] = m;
  }
  __syncthreads();
  float mt[IA];
#pragma unroll
  for (int i = 0; i < IA; ++i) {
    const float* sm = s_max + wm * 4 * R + 32 * i + rl;
    mt[i] = fmaxf(fmaxf(sm[0], sm[R]), fmaxf(sm[2 * R], sm[3 * R]));
  }
#pragma unroll
  for (int i = 0; i < IA; ++i) {
    float sum = 0.f;
#pragma unroll
    for (int j = 0; j < JB; ++j)
#pragma unroll
      for (int g = 0; g < 4; ++g)
#pragma unroll
        for (int q = 0; q < 4; ++q) sum += rnd<half_t>(expf(rnd<half_t>(logit(i, j, g, q) - mt[i])));
    sum += __shfl_xor(sum, 32, 64);
    if (h == 0) s_sum[(wm * 4 + wn) * R + 32 * i + rl] = sum;
    const int m = m0 + wm * R + 32 * i + rl;
    if (m < a.M) {  // the label's logit, from the one lane of the one tile holding it
      const long long c = a.ce.labels[m] - cb;
      if (c >= 0 && c < C && ((c >> 2) & 1) == h) {
        float v = 0.f;
#pragma unroll
        for (int j = 0; j < JB; ++j)
#pragma unroll
          for (int g = 0; g < 4; ++g)
#pragma unroll
            for (int q = 0; q < 4; ++q)
              if (c == 32 * j + 8 * g + 4 * h + q) v = logit(i, j, g, q);
        a.ce.label_logit[m] = v;
      }
    }
  }
  __syncthreads();
  if (wn == 0 && h == 0) {
    const int t = n0 / TN;
#pragma unroll
    for (int i = 0; i < IA; ++i) {
      const int m = m0 + wm * R + 32 * i + rl;
      const float* ss = s_sum + wm * 4 * R + 32 * i + rl;
      if (m < a.M)
        a.ce.part[static_cast<size_t>(m) * a.ce.tiles_n + t] =
            make_float2(mt[i], ((ss[0] + ss[R]) + ss[2 * R]) + ss[3 * R]);
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
  {  // written out: a loop here is not always unrolled, and acc must stay in registers
    const int na = n0 + wn * 64 + (lane & 31), nb = na + 32;
    const float ba = bias_at<EPI>(a, na), bb = bias_at<EPI>(a, nb);
    const int mb = m0 + wm * 64 + 4 * (lane >> 5);
    epilogue_tile32<EPI>(a, mb, na, acc[0][0], ba);
    epilogue_tile32<EPI>(a, mb, nb, acc[0][1], bb);
    epilogue_tile32<EPI>(a, mb + 32, na, acc[1][0], ba);
    epilogue_tile32<EPI>(a, mb + 32, nb, acc[1][1], bb);
  }
}

// ------------------------------------------------ fp16 MFMA GEMM, 256×256 block tile
// For large M·N (prefill, compute_loss): a 512-lane workgroup owns a 256×256 tile; its
// 8 waves (2×4, two per SIMD) each own 128×64 = 4×2 MFMA 32×32×16 tiles (128 fp32
// accumulators), so each A fragment read from LDS feeds 2 MFMAs and each B fragment 4.
// The main loop (stages of 64 k-columns double-buffered in 128 KiB of LDS by
// direct-to-LDS loads) is big::mainloop. Tiles are ordered XCD by XCD (workgroup b runs
// on XCD b % 8 and takes a contiguous range of tiles), grouped GM m-bands at a time so
// the workgroups resident on one XCD share A bands and B tiles in its L2.
constexpr int kHM = 256, kHN = 256, kHK = big::kK;
static_assert(kHN == kLinearCETile, "EPI_CE partials are per 256-column tile");
constexpr int kHT = big::kThreads;

template <int EPI, int GM, int TM, int TN>
__global__ __launch_bounds__(kHT, TM == 256 ? 1 : 4) void gemm_f16_big_kernel(LinearArgs a, int tiles_n, int tiles) {
  extern __shared__ __attribute__((aligned(1024))) char lds_raw[];
  constexpr int IA = TM / 64, JB = TN / 128;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
  const int wm = wave >> 2, wn = wave & 3;  // 2 × 4 waves of TM/2 × TN/4
  // XCD-aware tile order, GM m-bands per group
  const int t = big::xcd_tile(blockIdx.x, tiles);
  const int tiles_m = tiles / tiles_n;
  const int group = t / (GM * tiles_n), first = group * GM;
  const int gm = tiles_m - first < GM ? tiles_m - first : GM;
  const int in = t - group * GM * tiles_n;
  const int m0 = (first + in % gm) * TM, n0 = (in / gm) * TN;

  floatx16 acc[IA][JB];
#pragma unroll
  for (int i = 0; i < IA; ++i)
#pragma unroll
    for (int j = 0; j < JB; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
  if constexpr (EPI == EPI_BIAS_GELU && TM == 256) {
    // the tanh table into LDS past the staging region, 1 KiB per direct-to-LDS load (two
    // per wave); the main loop's first stage wait (vmcnt(0), then a barrier) publishes it
    static_assert(kTanhBytes == 16 * 1024, "two 1 KiB blocks per wave");
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int blk = 2 * wave + j;
      __builtin_amdgcn_global_load_lds(
          (const __attribute__((address_space(1))) void*)(g_tanh_tab + blk * 512 + lane * 8),
          (__attribute__((address_space(3))) void*)(lds_raw + Staged<TM, TN>::Lds + blk * 1024), 16, 0, 0);
    }
  }
  big::mainloop<TM, TN, true>(static_cast<const half_t*>(a.x), a.lda, static_cast<const half_t*>(a.w), a.K,
                              a.M, a.N, 0, a.K / kHK, m0, n0, lds_raw, acc);

  if constexpr (EPI == EPI_CE)
    epilogue_ce<TM, TN>(a, m0, n0, acc, lds_raw);
  else
    epilogue_staged<EPI, TM, TN>(a, m0, n0, acc, lds_raw);
}

template <int EPI, int GM, int TM, int TN>
int gemm_big_launch_gm(const LinearArgs& a, hipStream_t st) {
  static bool attr = false;
  // main loop: 128 KiB (256 × 256) or 64 KiB (128 × 128); epilogue: 144 KiB or 36 KiB;
  // 256 × 256 GELU: 16 KiB more for the tanh table (160 KiB, all of a CU's LDS)
  constexpr size_t lds = (big::Shape<TM, TN>::Lds > Staged<TM, TN>::Lds ? big::Shape<TM, TN>::Lds
                                                                        : Staged<TM, TN>::Lds) +
                         (EPI == EPI_BIAS_GELU && TM == 256 ? kTanhBytes : 0);
  if constexpr (EPI == EPI_BIAS_GELU && TM == 256) NML_TRY(ensure_tanh_tab(st));
  if (!attr) {
    NML_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(&gemm_f16_big_kernel<EPI, GM, TM, TN>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)));
    attr = true;
  }
  const int tiles_n = (a.N + TN - 1) / TN, tiles_m = (a.M + TM - 1) / TM;
  const int tiles = tiles_n * tiles_m;
  gemm_f16_big_kernel<EPI, GM, TM, TN><<<tiles, kHT, lds, st>>>(a, tiles_n, tiles);
  NML_LAUNCHED();
  return 0;
}

// 256 × 256 tiles where they fill the chip (≥ 256 of them), else 128 × 128 tiles on the
// same main loop (two workgroups per CU).
bool big_gemm_wide(const LinearArgs& a) {
  const long long tm = (a.M + kHM - 1) / kHM, tn = (a.N + kHN - 1) / kHN;
  return a.M >= 1024 && (tm * tn) % 8 == 0 && tm * tn >= 256;
}

// 256×256 tiles run one workgroup per CU, 128×128 tiles two, at ~1.2× the time per flop.
// Where the last round of 256 big tiles would be short (e.g. 280 tiles: two rounds, the
// second 9 % full) the small tiles finish first: 0.6·⌈t/128⌉ against ⌈t/256⌉ rounds of
// one big tile's time. C4's ragged prefill, N = 1024 at ~18k rows: 168 → 145 µs.
bool big_tiles_pay(const LinearArgs& a) {
  if (!big_gemm_wide(a)) return false;
  const long long t = ((a.M + kHM - 1) / kHM) * ((a.N + kHN - 1) / kHN);
  return 3 * ((t + 127) / 128) >= 5 * ((t + 255) / 256);
}

template <int EPI>
int gemm_big_launch(const LinearArgs& a, hipStream_t st) {
  if (!big_tiles_pay(a)) return gemm_big_launch_gm<EPI, 4, 128, 128>(a, st);
  const char* e = std::getenv("NIMBLEML_BIG_GM");
  const int gm = e ? atoi(e) : 4;
  if (gm == 1) return gemm_big_launch_gm<EPI, 1, kHM, kHN>(a, st);
  if (gm == 8) return gemm_big_launch_gm<EPI, 8, kHM, kHN>(a, st);
  return gemm_big_launch_gm<EPI, 4, kHM, kHN>(a, st);
}

// The direct-to-LDS kernels: K a multiple of 64, 16-byte aligned rows, and enough rows
// for 128-row tiles to be mostly full.
bool big_gemm_applies(const LinearArgs& a) {
  if (std::getenv("NIMBLEML_BIG_GEMM") && std::getenv("NIMBLEML_BIG_GEMM")[0] == '0') return false;
  if (a.K % kHK != 0 || a.lda % 8 != 0 || (reinterpret_cast<uintptr_t>(a.x) & 15) != 0) return false;
  if (big_gemm_wide(a)) return true;
  return a.M >= 256 && !(std::getenv("NIMBLEML_BIG_GEMM") && std::getenv("NIMBLEML_BIG_GEMM")[0] == 'w');
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

// ------------------------------------------------------- skinny MFMA GEMM (fp16)
// 8 < M ≤ 64 rows (batched decode): HBM-bound on W, so the grid is spread over N and,
// when N is small, over K. A workgroup owns 16 output columns (rows of W) for all M
// rows and one of S slices of K; its 4 waves take a quarter of the slice each and run
// v_mfma_f32_16x16x32_f16 with A = those 16 rows of W and B = 16 rows of x per m-tile
// (MT tiles). The quarters are summed through LDS in a fixed order. With S > 1,
// slices 0..S-2 publish their fp32 tile as 64-bit
// (1 << 32 | value) slots with relaxed device-scope stores (no cache-flushing fences);
// slice S-1 — dispatched after every other workgroup of the grid, so its bounded
// wait always ends — polls them, sums the slices in order (independent of arrival
// order), clears the slots for the next launch and runs the epilogue.
// Operand layout of the 16x16x32 MFMA: lane l holds A[l%16][(l/16)·8 + 0..7] and
// B[(l/16)·8 + 0..7][l%16]; the result D[(l/16)·4 + e][l%16], e < 4.
//
// NORM (decode RMSNorm fused into the GEMM that consumes it, kernels/fused_rmsnorm.py:
// 153-162): the producer of x (an EPI_BIAS_RESID GEMM) also wrote the sums of
// squares rnd(v·v) of its rounded outputs per 16-column piece (ssq_out); this kernel
// sums a row's pieces in a fixed order, takes inv = rnd(1 / sqrt(mean + eps)) and
// normalises each loaded x piece as rnd(rnd(x·inv)·g) with two fp16 multiplies — the
// rounding points of the separate RMSNorm kernel.
constexpr int kSkN = 16;

struct SkinnyWs {
  unsigned long long* part = nullptr;  // [tile][slice < S-1][MT·256] flagged partials, zero between launches
  size_t part_slots = 0;
  int tiles = 0;
};
// One workspace per library stream (the second serves work forked onto stream2), so
// split-K launches on the two streams never share partial slots.
SkinnyWs g_skinny_ws[2];
inline SkinnyWs& skinny_ws(hipStream_t st) { return g_skinny_ws[is_stream2(st) ? 1 : 0]; }

template <int EPI, int MT, int U, bool NORM>
__global__ __launch_bounds__(256) void skinny_f16_kernel(LinearArgs a, unsigned long long* ws) {
#pragma clang fp contract(off)
  __shared__ float red[4][MT][16][17];
  const half_t* __restrict__ X = static_cast<const half_t*>(a.x);
  const half_t* __restrict__ W = static_cast<const half_t*>(a.w);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int tile = blockIdx.x, n0 = tile * kSkN;
  const int S = gridDim.y, slice = blockIdx.y;
  const int M = a.M, N = a.N, K = a.K;
  const int kq = K / (4 * S);
  const int kbeg = (slice * 4 + wave) * kq;
  const int r = lane & 15, kk = (lane >> 4) * 8;
  const bool nvalid = n0 + r < N;
  const half_t* wp = W + static_cast<long long>(nvalid ? n0 + r : 0) * K + kbeg + kk;
  const half_t* xp[MT];
  bool mvalid[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) {
    const int m = t * 16 + r;
    mvalid[t] = m < M;
    xp[t] = X + static_cast<long long>(mvalid[t] ? m : 0) * a.lda + kbeg + kk;
  }
  floatx4 acc[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) acc[t] = floatx4{0.f, 0.f, 0.f, 0.f};
  const half8 z8 = {0, 0, 0, 0, 0, 0, 0, 0};
  // The epilogue's bias and residual (written before this launch) are loaded now, in
  // the same round trip as the operands, by the workgroup that stores the output.
  // Addresses are clamped in bounds and the loads unconditional, so that no wait for
  // them is forced where branches join.
  const int ej = threadIdx.x >> 4, ei = threadIdx.x & 15;
  const int ec = n0 + ei < N ? n0 + ei : N - 1;
  float pre_b = 0.f, pre_r[MT];
  if constexpr (EPI != EPI_NONE) pre_b = static_cast<float>(static_cast<const half_t*>(a.bias)[ec]);
  // EPI_QKV: the row's cache position (pos_base) is loaded here too, and the destination
  // of each output (q, or the K/V cache row) is formed below while the operands are in
  // flight, not after them.
  int pre_pos[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) {
    pre_r[t] = 0.f;
    pre_pos[t] = 0;
    const int m = t * 16 + ej < M ? t * 16 + ej : M - 1;
    if constexpr (EPI == EPI_BIAS_RESID)
      pre_r[t] = static_cast<float>(static_cast<const half_t*>(a.resid)[static_cast<size_t>(m) * N + ec]);
    if constexpr (EPI == EPI_QKV) {
      const QKVDst& q = a.qkv;
      int b = m;  // row segments: (b << 16) | s; else b = m / S
      if (q.row_seg) b = q.row_seg[m] >> 16;
      else if (q.S != 1) b = m / q.S;
      pre_pos[t] = q.pos_base ? q.pos_base[b] : 0;
    }
  }
  // Operands of one step of U 32-wide k blocks (and the RMSNorm gains with NORM); the
  // first step shares its round trip with the RMSNorm statistics.
  half8 av[U], bv[U][MT], gv[U];
  const half_t* gp = NORM ? static_cast<const half_t*>(a.norm_g) + kbeg + kk : nullptr;
  auto load = [&](int k) {
#pragma unroll
    for (int u = 0; u < U; ++u) {  // wp, xp point at row 0 where invalid: zeroed after
      const half8 w8 = *reinterpret_cast<const half8*>(wp + k + u * 32);
      av[u] = nvalid ? w8 : z8;
#pragma unroll
      for (int t = 0; t < MT; ++t) {
        const half8 x8 = *reinterpret_cast<const half8*>(xp[t] + k + u * 32);
        bv[u][t] = mvalid[t] ? x8 : z8;
      }
      if constexpr (NORM) gv[u] = *reinterpret_cast<const half8*>(gp + k + u * 32);
    }
  };
  // RMSNorm statistics (NORM): lane group g = lane / 16 sums the g-th quarter of the
  // K/16 pieces of rows t·16 + r in order; the quarters are added as (q0 + q1) + (q2 + q3)
  // by lane exchanges (the same value in all four groups). With K = 1024 the loads are
  // issued before the operands': they return first, and the statistics are formed while
  // the operands are in flight. No barrier.
  const int np = K / 16, nq4 = np / 4, g = lane >> 4;
  float sqs[MT];
  const float* sps[MT];
  floatx4 v4[MT][4];
  if constexpr (NORM) {
#pragma unroll
    for (int t = 0; t < MT; ++t) {  // rows clamped to 0 past M (their result is discarded)
      const int row = t * 16 + r;
      sps[t] = a.ssq_in + static_cast<size_t>(row < M ? row : 0) * np + g * nq4;
      sqs[t] = 0.f;
    }
    if (nq4 == 16) {
#pragma unroll
      for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int e = 0; e < 4; ++e) v4[t][e] = *reinterpret_cast<const floatx4*>(sps[t] + 4 * e);
    }
  }
  load(0);
  half8 inv8[MT];
  if constexpr (NORM) {
    if (nq4 == 16) {  // K = 1024: every tile's quarter in one batch of 16-byte loads
#pragma unroll
      for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int e = 0; e < 4; ++e)
#pragma unroll
          for (int c = 0; c < 4; ++c) sqs[t] += v4[t][e][c];
    } else {
#pragma unroll
      for (int t = 0; t < MT; ++t)
        for (int j = 0; j < nq4; j += 2) {  // nq4 is even: K is a multiple of 128
          const float2 v2 = *reinterpret_cast<const float2*>(sps[t] + j);
          sqs[t] += v2.x;
          sqs[t] += v2.y;
        }
    }
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      const int row = t * 16 + r;
      float sq = sqs[t];
      sq += __shfl_xor(sq, 16, 64);
      sq += __shfl_xor(sq, 32, 64);
      float inv = 0.f;  // rows past M load zeros and stay zero
      if (row < M) inv = rnd<half_t>(1.0f / sqrtf(sq / static_cast<float>(K) + a.norm_eps));
      const half_t hv = static_cast<half_t>(inv);
      inv8[t] = half8{hv, hv, hv, hv, hv, hv, hv, hv};
    }
  }
  half_t* qdst[MT];
  if constexpr (EPI == EPI_QKV) {
    const QKVDst& q = a.qkv;
    const int which = ec / q.d, within = ec - which * q.d;
    const int hd = within / q.dk, j = within - hd * q.dk;
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      const int m = t * 16 + ej < M ? t * 16 + ej : M - 1;
      int b = m, sp = 0;
      if (q.row_seg) {
        const int rs = q.row_seg[m];
        b = rs >> 16;
        sp = rs & 0xffff;
      } else if (q.S != 1) {
        b = m / q.S;
        sp = m - b * q.S;
      }
      qdst[t] = which == 0
          ? static_cast<half_t*>(q.q) + ((static_cast<size_t>(b) * q.H + hd) * q.S + sp) * q.dk + j
          : static_cast<half_t*>(which == 1 ? q.k : q.v) + b * q.kv_stride_b + hd * q.kv_stride_h +
                static_cast<long long>(pre_pos[t] + sp) * q.dk + j;
      asm volatile("" ::"v"(qdst[t]));  // formed here, before the operands are waited for
    }
  }
  for (int k = 0; k < kq; k += 32 * U) {
    if constexpr (NORM) {
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int t = 0; t < MT; ++t) bv[u][t] = (bv[u][t] * inv8[t]) * gv[u];
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int t = 0; t < MT; ++t)
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[u], bv[u][t], acc[t], 0, 0, 0);
    if (k + 32 * U < kq) load(k + 32 * U);
  }
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int e = 0; e < 4; ++e) red[wave][t][(lane >> 4) * 4 + e][lane & 15] = acc[t][e];
  __syncthreads();
  // thread → outputs o = tid + 256·t: (t, j = m within the tile, i = W row within the tile)
  float sum[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) {
    const int j = threadIdx.x >> 4, i = threadIdx.x & 15;
    sum[t] = ((red[0][t][i][j] + red[1][t][i][j]) + red[2][t][i][j]) + red[3][t][i][j];
  }
  if (S > 1) {
    typedef unsigned long long u64;
    u64* tile_ws = ws + static_cast<size_t>(tile) * (S - 1) * (MT * 256);
    if (slice < S - 1) {
#pragma unroll
      for (int t = 0; t < MT; ++t)
        __hip_atomic_store(tile_ws + (static_cast<size_t>(slice) * MT + t) * 256 + threadIdx.x,
                           (1ull << 32) | __float_as_uint(sum[t]), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
      return;
    }
    float tot[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) tot[t] = 0.f;
    for (int q = 0; q < S - 1; ++q) {
#pragma unroll
      for (int t = 0; t < MT; ++t) {
        u64* sl = tile_ws + (static_cast<size_t>(q) * MT + t) * 256 + threadIdx.x;
        u64 v = __hip_atomic_load(sl, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        for (unsigned spins = 0; (v >> 32) == 0 && spins < (1u << 22); ++spins) {
          __builtin_amdgcn_s_sleep(1);
          v = __hip_atomic_load(sl, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        tot[t] += __uint_as_float(static_cast<uint32_t>(v));
        // consumed: clear for the next launch, through the same device-coherent path
        __hip_atomic_store(sl, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
#pragma unroll
    for (int t = 0; t < MT; ++t) sum[t] = tot[t] + sum[t];
  }
#pragma unroll
  for (int t = 0; t < MT; ++t) {
    const int j = ej, i = ei;
    const int m = t * 16 + j, n = n0 + i;
    float v = 0.f;
    if constexpr (EPI == EPI_QKV) {
      if (m < M && n < N) {
        v = rnd<half_t>(rnd<half_t>(sum[t]) + pre_b);
        *qdst[t] = static_cast<half_t>(v);
      }
    } else if (m < M && n < N) {
      v = epilogue_with<half_t, EPI>(a, m, n, sum[t], pre_b, pre_r[t]);
    }
    if constexpr (EPI == EPI_BIAS_RESID) {
      if (a.ssq_out) {  // this tile's piece of the row's sum of squares (16 lanes = 1 row)
        const float sq = row16_sum_dpp(rnd<half_t>(v * v));
        if (i == 0 && m < M) a.ssq_out[static_cast<size_t>(m) * (N / kSkN) + tile] = sq;
      }
    }
  }
}

// Slices of K: about 1024 columns of K per workgroup (measured on MI355X with weights
// streamed from HBM: unsplit is fastest for K = 1024 at N = 1024…4096, four slices for
// K = 4096), each wave's part of K a multiple of 32, and a workspace large enough.
int skinny_slices(const LinearArgs& a, int MT, const SkinnyWs& w) {
  const int tiles = (a.N + kSkN - 1) / kSkN;
  int S = 1;
  while (S < 8 && a.K / S > 1024 && a.K % (128 * S * 2) == 0) S *= 2;
  while (S > 1 && (tiles > w.tiles || static_cast<size_t>(tiles) * (S - 1) * MT * 256 > w.part_slots))
    S /= 2;
  return S;
}

template <int EPI, int MT, bool NORM>
int skinny_launch(const LinearArgs& a, hipStream_t st) {
  const SkinnyWs& w = skinny_ws(st);
  const int S = skinny_slices(a, MT, w);
  dim3 grid((a.N + kSkN - 1) / kSkN, S);
  const int kq = a.K / (4 * S);
  unsigned long long* ws = w.part;
  if (kq == 256)  // every operand of the wave in one round trip
    skinny_f16_kernel<EPI, MT, 8, NORM><<<grid, 256, 0, st>>>(a, ws);
  else if (kq % 128 == 0)
    skinny_f16_kernel<EPI, MT, 4, NORM><<<grid, 256, 0, st>>>(a, ws);
  else if (kq % 64 == 0)
    skinny_f16_kernel<EPI, MT, 2, NORM><<<grid, 256, 0, st>>>(a, ws);
  else
    skinny_f16_kernel<EPI, MT, 1, NORM><<<grid, 256, 0, st>>>(a, ws);
  NML_LAUNCHED();
  return 0;
}

// ------------------------------------------------ wide skinny GEMM (tied head, decode)
// 8 < M ≤ 64 rows against a wide W (the tied LM head: V rows), no epilogue. The skinny
// kernel above reads all of x for every 16 W rows (at M = 32 that is twice the bytes of
// W it streams), so here a workgroup stages the M rows of x in LDS once — with the fused
// RMSNorm applied on the way, the skinny kernel's statistics and rounding — and each of
// its 4 waves streams 16 W rows over the whole K: v_mfma_f32_16x16x32_f16 with A = the
// 16 W rows (all K/32 k-blocks of a wave in flight in two batches of 16) and B = 16 x
// rows per m-tile from LDS. Every output element is one wave's sum over k in order.
// (C4's tied head, 32 × 1024 against 32000 rows: 34.3 → 20.5 µs.)
constexpr int kWideCols = 64;  // W rows per workgroup

template <int MT>
constexpr size_t wide_lds(int K) {
  return static_cast<size_t>(MT) * 16 * (K + 8) * sizeof(half_t) + MT * 16 * sizeof(float);
}

template <int MT, bool NORM>
__global__ __launch_bounds__(256, 2) void skinny_wide_kernel(LinearArgs a) {
  extern __shared__ __attribute__((aligned(16))) char lds_w[];
  const int K = a.K, M = a.M, N = a.N, P = K + 8;  // x rows 16 bytes apart in bank space
  half_t* xs = reinterpret_cast<half_t*>(lds_w);
  float* s_inv = reinterpret_cast<float*>(lds_w + static_cast<size_t>(MT) * 16 * P * sizeof(half_t));
  const half_t* __restrict__ X = static_cast<const half_t*>(a.x);
  const half_t* __restrict__ W = static_cast<const half_t*>(a.w);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n0 = blockIdx.x * kWideCols + wave * 16;
  const int r = lane & 15, kk = (lane >> 4) * 8;
  // this lane's W row (clamped; rows past N are computed and not stored)
  const half_t* wp = W + static_cast<long long>(n0 + r < N ? n0 + r : N - 1) * K + kk;
  const int nb = K / 32;
  half8 w0[16], w1[16];
  auto load = [&](half8 (&w)[16], int b0) {
#pragma unroll
    for (int u = 0; u < 16; ++u) w[u] = *reinterpret_cast<const half8*>(wp + (b0 + u) * 32);
  };
  load(w0, 0);  // the weights' round trip overlaps the staging of x
  if (nb > 16) load(w1, 16);
  if constexpr (NORM) {
    // 4 lanes per row, lane g summing the g-th quarter of the row's K/16 pieces in order,
    // the quarters added as (q0 + q1) + (q2 + q3)
    if (tid < MT * 64) {
      const int row = tid >> 2, g = tid & 3, np = K / 16, nq4 = np / 4;
      float q = 0.f;
      if (row < M) {
        const float* sp = a.ssq_in + static_cast<size_t>(row) * np + g * nq4;
        for (int j = 0; j < nq4; ++j) q += sp[j];
      }
      q += __shfl_xor(q, 1, 64);
      q += __shfl_xor(q, 2, 64);
      if (g == 0)
        s_inv[row] = row < M ? rnd<half_t>(1.0f / sqrtf(q / static_cast<float>(K) + a.norm_eps)) : 0.f;
    }
    __syncthreads();
  }
  const half8 z8 = {0, 0, 0, 0, 0, 0, 0, 0};
  const int cpr = K / 8;  // 8-element chunks per row
  for (int c = tid; c < MT * 16 * cpr; c += 256) {
    const int row = c / cpr, col = (c - row * cpr) * 8;
    half8 v = row < M ? *reinterpret_cast<const half8*>(X + static_cast<long long>(row) * a.lda + col) : z8;
    if constexpr (NORM) {
      const half_t hv = static_cast<half_t>(s_inv[row]);
      const half8 inv8 = {hv, hv, hv, hv, hv, hv, hv, hv};
      v = (v * inv8) * *reinterpret_cast<const half8*>(static_cast<const half_t*>(a.norm_g) + col);
    }
    *reinterpret_cast<half8*>(xs + row * P + col) = v;
  }
  __syncthreads();
  floatx4 acc[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) acc[t] = floatx4{0.f, 0.f, 0.f, 0.f};
  auto mma = [&](const half8 (&w)[16], int b0) {
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const int k = (b0 + u) * 32 + kk;
#pragma unroll
      for (int t = 0; t < MT; ++t) {
        const half8 xb = *reinterpret_cast<const half8*>(xs + (16 * t + r) * P + k);
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(w[u], xb, acc[t], 0, 0, 0);
      }
    }
  };
  for (int b0 = 0; b0 < nb; b0 += 32) {
    mma(w0, b0);
    if (b0 + 32 < nb) load(w0, b0 + 32);
    if (b0 + 16 < nb) {
      mma(w1, b0 + 16);
      if (b0 + 48 < nb) load(w1, b0 + 48);
    }
  }
  // lane: rows n0 + 4·(lane/16) + e of W (output columns), x row 16t + lane%16
  half_t* out = static_cast<half_t*>(a.out);
  const int nc = n0 + 4 * (lane >> 4);
#pragma unroll
  for (int t = 0; t < MT; ++t) {
    const int m = 16 * t + r;
    if (m >= M) continue;
    half4 h;
#pragma unroll
    for (int e = 0; e < 4; ++e) h[e] = static_cast<half_t>(acc[t][e]);
    half_t* o = out + static_cast<size_t>(m) * N + nc;
    if (nc + 3 < N && (N & 3) == 0) {
      *reinterpret_cast<half4*>(o) = h;
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (nc + e < N) o[e] = h[e];
    }
  }
}

template <int MT, bool NORM>
int skinny_wide_launch(const LinearArgs& a, hipStream_t st) {
  static bool attr = false;
  const size_t lds = wide_lds<MT>(a.K);
  if (!attr) {
    NML_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(&skinny_wide_kernel<MT, NORM>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, 80 * 1024));
    attr = true;
  }
  skinny_wide_kernel<MT, NORM><<<(a.N + kWideCols - 1) / kWideCols, 256, lds, st>>>(a);
  NML_LAUNCHED();
  return 0;
}

// The wide kernel for head-like shapes: many W rows, no epilogue, K a multiple of 512,
// x rows 16-byte aligned, and two workgroups' x in LDS.
bool skinny_wide_applies(const LinearArgs& a, int MT) {
  return a.epi == EPI_NONE && a.N >= 8192 && a.K % 512 == 0 && a.lda % 8 == 0 &&
         static_cast<size_t>(MT) * 16 * (a.K + 8) * sizeof(half_t) + MT * 16 * sizeof(float) <=
             80 * 1024;
}

template <int EPI, int MT>
int skinny_dispatch_u(const LinearArgs& a, hipStream_t st) {
  if constexpr (EPI == EPI_NONE) {
    if (skinny_wide_applies(a, MT))
      return a.ssq_in ? skinny_wide_launch<MT, true>(a, st) : skinny_wide_launch<MT, false>(a, st);
  }
  if (a.ssq_in) {
    if constexpr (EPI == EPI_NONE || EPI == EPI_BIAS_GELU || EPI == EPI_QKV)
      return skinny_launch<EPI, MT, true>(a, st);
    set_error("linear: fused RMSNorm is not available with epilogue %d", EPI);
    return -1;
  }
  return skinny_launch<EPI, MT, false>(a, st);
}

template <int EPI>
int skinny_dispatch(const LinearArgs& a, hipStream_t st) {
  switch ((a.M + 15) / 16) {
    case 1: return skinny_dispatch_u<EPI, 1>(a, st);
    case 2: return skinny_dispatch_u<EPI, 2>(a, st);
    case 3: return skinny_dispatch_u<EPI, 3>(a, st);
    default: return skinny_dispatch_u<EPI, 4>(a, st);
  }
}

bool skinny_applies(int dt, int M, int K) { return dt == F16 && M > 8 && M <= 64 && K % 128 == 0; }

template <typename T, int EPI>
int linear_typed(const LinearArgs& a, hipStream_t st) {
  if constexpr (sizeof(T) == 2) {
    if (skinny_applies(F16, a.M, a.K)) return skinny_dispatch<EPI>(a, st);
  }
  if (a.ssq_in || a.ssq_out) {
    set_error("linear: fused RMSNorm needs the fp16 skinny path (8 < rows <= 64)");
    return -1;
  }
  if (a.M <= 8) {
    if (a.M <= 1) return gemv_dispatch_rpw<T, EPI, 1>(a, st);
    if (a.M <= 2) return gemv_dispatch_rpw<T, EPI, 2>(a, st);
    if (a.M <= 4) return gemv_dispatch_rpw<T, EPI, 4>(a, st);
    return gemv_dispatch_rpw<T, EPI, 8>(a, st);
  }
  if constexpr (sizeof(T) == 2) {
    if (big_gemm_applies(a)) return gemm_big_launch<EPI>(a, st);
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
    case EPI_CE:
      if constexpr (sizeof(T) == 2) return gemm_big_launch_gm<EPI_CE, 4, kHM, kHN>(a, st);
      break;
  }
  set_error("unknown epilogue %d", a.epi);
  return -1;
}

}  // namespace

int linear_reserve_workspace(int max_n) {
  // Flagged split-K partials for up to 8 slices of 64 rows at N = max_n (16-column
  // tiles), zeroed. Grow-only; call outside stream capture.
  const int tiles = (max_n + kSkN - 1) / kSkN;
  const size_t slots = static_cast<size_t>(tiles) * 7 * 4 * 256;
  for (SkinnyWs& w : g_skinny_ws) {
    if (tiles <= w.tiles && slots <= w.part_slots) continue;
    NML_HIP(hipDeviceSynchronize());  // both streams may hold launches that use it
    if (w.part) NML_HIP(hipFree(w.part));
    w = SkinnyWs{};
    unsigned long long* p = nullptr;
    NML_HIP(hipMalloc(&p, slots * 8));
    NML_HIP(hipMemset(p, 0, slots * 8));
    w.part = p;
    w.part_slots = slots;
    w.tiles = tiles;
  }
  return 0;
}

int launch_linear(int dt, const LinearArgs& a, hipStream_t st) {
  if (a.M == 0 || a.N == 0) return 0;
  const int vec = dt == F16 ? 8 : 4;
  NML_REQUIRE(a.K > 0 && a.K % vec == 0, "linear: K=%d must be a positive multiple of %d", a.K, vec);
  NML_REQUIRE(a.lda % vec == 0, "linear: row stride %lld must be a multiple of %d", a.lda, vec);
  NML_REQUIRE((reinterpret_cast<uintptr_t>(a.x) & 15) == 0 &&
                  (reinterpret_cast<uintptr_t>(a.w) & 15) == 0,
              "linear: x and w must be 16-byte aligned");
  NML_REQUIRE(a.epi == EPI_NONE || a.epi == EPI_CE || a.bias != nullptr,
              "linear: epilogue %d needs a bias", a.epi);
  NML_REQUIRE(a.epi != EPI_CE ||
                  (linear_ce_fusable(dt, a.M, a.K, a.N) && a.lda == a.K && a.ce.labels &&
                   a.ce.part && a.ce.label_logit && a.ce.tiles_n == (a.N + kHN - 1) / kHN),
              "linear: the fused cross-entropy epilogue needs fp16, 256 x 256 tiles and its outputs");
  NML_REQUIRE(a.epi != EPI_BIAS_RESID || a.resid != nullptr, "linear: residual pointer missing");
  NML_REQUIRE(a.epi != EPI_QKV || (a.qkv.d > 0 && a.qkv.dk > 0 && a.N == 3 * a.qkv.d &&
                                   (a.qkv.row_seg || a.M == a.qkv.S * (a.M / a.qkv.S))),
              "linear: bad QKV destination");
  NML_REQUIRE(!a.ssq_in || (a.norm_g != nullptr && linear_norm_fusable(dt, a.M, a.K, a.N)),
              "linear: fused RMSNorm needs a gain and the fp16 skinny shape");
  NML_REQUIRE(!a.pre_out || (a.epi == EPI_BIAS_GELU && a.M > 64),
              "linear: the pre-activation copy needs the GELU epilogue and more than 64 rows");
  NML_REQUIRE(!a.ssq_out || (a.epi == EPI_BIAS_RESID && linear_norm_fusable(dt, a.M, a.K, a.N)),
              "linear: sums of squares are written by an fp16 skinny residual GEMM only");
  return dt == F16 ? linear_epi<half_t>(a, st) : linear_epi<float>(a, st);
}

bool linear_ce_fusable(int dt, int M, int K, int N) {
  LinearArgs t{};
  t.M = M;
  t.N = N;
  return dt == F16 && K % kHK == 0 && big_gemm_wide(t);
}

bool linear_norm_fusable(int dt, int M, int K, int N) {
  return skinny_applies(dt, M, K) && K % kSkN == 0 && N % kSkN == 0;
}

}  // namespace nml
