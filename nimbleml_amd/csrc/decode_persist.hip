// Persistent decode step for one sequence (batch 1): the whole token — embedding,
// L pre-norm blocks, final RMSNorm, tied LM head and the greedy choice — in ONE
// launch of 256 workgroups (one per CU), so the per-layer dependency latencies are
// paid as ~1 µs data exchanges instead of ~4 µs kernel boundaries, and each
// workgroup's weight loads for a phase are already in flight while it waits for
// that phase's inputs.
//
// Phases of layer l (neural_network/_fused_arrays.py:251-284; same rounding points
// as the multi-kernel path and the reference's separate NumPy ops):
//   P1  x → RMSNorm₁ → rows of [W_q|W_k|W_v]ᵀ + b → q, k, v of one head
//       (k, v also into the cache at `pos`)
//   P2  attention over 64-key chunks of the cache: (max, Σp, Σp·v) per chunk
//   P2b one workgroup per head merges its chunks → attention output of the head
//   P3  rows of W_oᵀ + b_o + residual → x_mid
//   P4  x_mid → RMSNorm₂ → rows of W₁ᵀ + b₁ → GELU → h
//   P5  rows of W₂ᵀ + b₂ + residual → x of layer l+1
// then RMSNorm_f → rows of the tied head (logits) with a per-workgroup argmax, and
// workgroup 0 makes the greedy choice (models/generate.py:40-41, first index on ties).
//
// Exchange: every value that crosses workgroups is written as one 64-bit slot
// (tag << 32 | payload) with a relaxed device-scope atomic store, and read with
// relaxed device-scope atomic loads until the tag matches. tag = epoch·(8L+8) +
// phase id, epoch = a per-launch counter kept on the device, so a slot written in an
// earlier phase or step never matches. Every wait is bounded: after ~0.5 s (or
// once another thread has given up) it sets bit 2 of *err and goes on, so the
// grid always drains and the host reports the failure.
//
// Work placement is XCD-aware: the dispatcher deals workgroups to the 8 XCDs round
// robin (workgroup g on XCD (g + c) % 8 for a per-launch offset c; measured c = 7), so the
// workgroups g ≡ x (mod 8) share one XCD, and a head's team — its QKV rows, attention
// chunks and merge — is made of such workgroups.
#include "kernels.hpp"

namespace nml {

namespace {

constexpr int kG = kPersistGroups;  // 256 workgroups
constexpr int kT = 256;             // 4 waves each
constexpr int kXcd = 8;
constexpr int kChunk = 64;          // keys per attention work item
constexpr int kMaxCh = kPersistMaxLen / kChunk;
constexpr unsigned kSpinLimit = 1u << 19;
constexpr int kLine = 16;           // 64-bit slots per 128-byte line

// Exchange-slot regions, in 64-bit slots. Each producing workgroup's slots start on a
// line of their own: lines shared by producers make their write-through stores and
// the consumers' polls of that line contend, which measured ~1.5x slower exchanges.
constexpr int lines_of(int slots) { return (slots + kLine - 1) / kLine * kLine; }

template <int D, int DK>
struct SlotLayout {
  static constexpr int H = D / DK, TEAM = kG / H, F = 4 * D;
  static constexpr int PCH = lines_of(DK + 2);   // one chunk's partial
  static constexpr int SX = lines_of(D / kG);    // per producer: D/kG values of x (x_mid)
  static constexpr int SQ = lines_of(3 * DK / TEAM);  // per team member: its QKV rows
  static constexpr int SH = lines_of(F / kG);    // per producer: F/kG values of h
  static constexpr int X = 0;
  static constexpr int QKV = X + kG * SX;
  static constexpr int ATT = QKV + H * TEAM * SQ;   // H × DK: attention output
  static constexpr int XM = ATT + H * DK;
  static constexpr int HID = XM + kG * SX;
  static constexpr int PART = HID + kG * SH;        // H·kMaxCh × PCH: chunk partials
  static constexpr int ARG = PART + H * kMaxCh * PCH;  // kG × line: (best, index)
  static constexpr int total = ARG + kG * kLine;
  static_assert(ATT % kLine == 0 && (DK / 2) % kLine == 0, "line-aligned heads");
};

typedef unsigned long long u64;

#define NML_MARK(k)                                                                 \
  do {                                                                              \
    if (trace && threadIdx.x == 0) trace[(k)] = wall_clock64();                    \
  } while (0)

template <typename T>
struct V16;
template <>
struct V16<half_t> {
  typedef half8 type;
  static constexpr int n = 8;
};
template <>
struct V16<float> {
  typedef floatx4 type;
  static constexpr int n = 4;
};

template <typename T>
__device__ __forceinline__ uint32_t enc(float v);
template <>
__device__ __forceinline__ uint32_t enc<float>(float v) { return __float_as_uint(v); }
template <>
__device__ __forceinline__ uint32_t enc<half_t>(float v) {
  return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<half_t>(v)));
}
template <typename T>
__device__ __forceinline__ T dec(uint32_t u);
template <>
__device__ __forceinline__ float dec<float>(uint32_t u) { return __uint_as_float(u); }
template <>
__device__ __forceinline__ half_t dec<half_t>(uint32_t u) {
  return __builtin_bit_cast(half_t, static_cast<uint16_t>(u));
}

__device__ __forceinline__ void put(u64* s, uint32_t tag, uint32_t payload) {
  __hip_atomic_store(s, (static_cast<u64>(tag) << 32) | payload, __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ u64 peek(const u64* s) {
  return __hip_atomic_load(const_cast<u64*>(s), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Spin bookkeeping shared by the waits: after kSpinLimit rounds, or once any thread
// of the grid has given up (bit 2 of *err), stop waiting.
__device__ __forceinline__ bool give_up(unsigned spins, int* err, int& bad) {
  if ((spins & 255u) != 255u) return false;
  const int e = __hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (spins > kSpinLimit || (e & 4)) {
    atomicOr(err, 4);
    bad = 1;
    return true;
  }
  return false;
}

// Payloads of slots[idx[j]] (j < N, idx[j] < 0 = none) once each carries `tag`. All
// loads are issued together and every retry re-issues the missing ones together, so
// a wait costs one round trip per retry, not one per slot.
template <int N>
__device__ __forceinline__ void wait_slots(const u64* slots, const int (&idx)[N], uint32_t tag,
                                           uint32_t (&out)[N], int* err, int& bad) {
  u64 v[N];
#pragma unroll
  for (int j = 0; j < N; ++j) v[j] = idx[j] >= 0 ? peek(slots + idx[j]) : (static_cast<u64>(tag) << 32);
  for (unsigned spins = 0;; ++spins) {
    bool all = true;
#pragma unroll
    for (int j = 0; j < N; ++j) all = all && static_cast<uint32_t>(v[j] >> 32) == tag;
    if (all || bad) break;
    if (give_up(spins, err, bad)) break;
    __builtin_amdgcn_s_sleep(1);
    // Reload every slot: one that already matched cannot move on to a newer tag
    // while this consumer has not finished with it.
#pragma unroll
    for (int j = 0; j < N; ++j)
      v[j] = idx[j] >= 0 ? peek(slots + idx[j]) : (static_cast<u64>(tag) << 32);
  }
#pragma unroll
  for (int j = 0; j < N; ++j) out[j] = static_cast<uint32_t>(v[j]);
}

// v[j] = slot p[j·stride] once every one carries `tag` (same retry scheme).
template <int N>
__device__ __forceinline__ void poll_batch(const u64* p, int stride, uint32_t tag, u64 (&v)[N],
                                           int* err, int& bad) {
#pragma unroll
  for (int j = 0; j < N; ++j) v[j] = peek(p + stride * j);
  for (unsigned spins = 0;; ++spins) {
    bool all = true;
#pragma unroll
    for (int j = 0; j < N; ++j) all = all && static_cast<uint32_t>(v[j] >> 32) == tag;
    if (all || bad) break;
    if (give_up(spins, err, bad)) break;
    __builtin_amdgcn_s_sleep(1);
#pragma unroll
    for (int j = 0; j < N; ++j) v[j] = peek(p + stride * j);
  }
}

// Values per exchange slot for the FFN hidden vector and the attention output: two
// fp16 values share one 32-bit payload (element 2k in the low half), fp32 takes one.
template <typename T>
constexpr int kPack = sizeof(T) == 2 ? 2 : 1;

template <typename T>
__device__ __forceinline__ uint32_t pack(float v0, float v1);
template <>
__device__ __forceinline__ uint32_t pack<float>(float v0, float) { return __float_as_uint(v0); }
template <>
__device__ __forceinline__ uint32_t pack<half_t>(float v0, float v1) {
  return enc<half_t>(v0) | (enc<half_t>(v1) << 16);
}

// Producer side: values v0, v1 of rows r, r+1 (r even) of a packed region.
template <typename T>
__device__ __forceinline__ void put_pair(u64* region, int r, uint32_t tag, float v0, float v1) {
  if constexpr (kPack<T> == 2) {
    put(region + r / 2, tag, pack<T>(v0, v1));
  } else {
    put(region + r, tag, pack<T>(v0, 0.f));
    put(region + r + 1, tag, pack<T>(v1, 0.f));
  }
}

// Store one slot payload (PK values) as element e of dst (LDS).
template <typename T, int PK>
__device__ __forceinline__ void sink_payload(T* dst, int e, uint32_t p) {
  if constexpr (PK == 2 || sizeof(T) == 4)
    reinterpret_cast<uint32_t*>(dst)[e / PK] = p;  // raw packed / fp32 payload
  else
    dst[e] = dec<T>(p);
}

// dst[0..N) from N / PK contiguous slots (a region whose producers own whole lines);
// thread t takes slots t, t+kT, ….
template <typename T, int N, int PK>
__device__ __forceinline__ void gather(const u64* slots, uint32_t tag, T* dst, int* err, int& bad) {
  constexpr int PER = N / PK / kT;
  static_assert(PER * PK * kT == N, "gather shape");
  u64 v[PER];
  poll_batch<PER>(slots + threadIdx.x, kT, tag, v, err, bad);
#pragma unroll
  for (int j = 0; j < PER; ++j)
    sink_payload<T, PK>(dst, (threadIdx.x + kT * j) * PK, static_cast<uint32_t>(v[j]));
}

// dst[0..NPROD·VP) from a region where producer p keeps its VP values in SP = VP / PK
// slots at p·LS + s (LS: whole lines). Thread t takes slot t % SP of producers t / SP,
// t / SP + kT/SP, …, so each wave's load instruction reads whole producer lines.
template <typename T, int NPROD, int VP, int PK, int LS>
__device__ __forceinline__ void gather_lines(const u64* region, uint32_t tag, T* dst, int* err,
                                             int& bad) {
  constexpr int SP = VP / PK;
  static_assert(SP <= LS && 64 % SP == 0, "slots per producer");
  constexpr int PPR = kT / SP;  // producers per round of the block's threads
  constexpr int PER = NPROD / PPR;
  static_assert(NPROD % PPR == 0, "gather shape");
  const int sl = threadIdx.x % SP, pq = threadIdx.x / SP;
  u64 v[PER];
  poll_batch<PER>(region + pq * LS + sl, PPR * LS, tag, v, err, bad);
#pragma unroll
  for (int j = 0; j < PER; ++j)
    sink_payload<T, PK>(dst, (pq + PPR * j) * VP + sl * PK, static_cast<uint32_t>(v[j]));
}

// The chunk partials of one head (chunks c < nch; at slot c·PCH + k: the chunk's max
// (k = 0), sum (1) and DK weighted value sums (2…)) into dst[c·(DK+2) + k]. Wave w
// takes chunks w, w+4, …; its lane l waits for value sum l of each, lanes 0 and 1 also
// for the max and the sum; 8 chunks per wave per round.
template <int DK, int PCH>
__device__ __forceinline__ void gather_partials(const u64* src, int nch, uint32_t tag, float* dst,
                                                int* err, int& bad) {
  static_assert(DK == 64 && kT == 256, "one lane per value sum, four waves");
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
  const u64 want = static_cast<u64>(tag) << 32;
  for (int c0 = w; c0 < nch; c0 += 32) {
    u64 v[8], m[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int c = c0 + 4 * j;
      v[j] = c < nch ? peek(src + c * PCH + 2 + l) : want;
      m[j] = (c < nch && l < 2) ? peek(src + c * PCH + l) : want;
    }
    for (unsigned spins = 0;; ++spins) {
      bool all = true;
#pragma unroll
      for (int j = 0; j < 8; ++j)
        all = all && static_cast<uint32_t>(v[j] >> 32) == tag &&
              static_cast<uint32_t>(m[j] >> 32) == tag;
      if (all || bad) break;
      if (give_up(spins, err, bad)) break;
      __builtin_amdgcn_s_sleep(1);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int c = c0 + 4 * j;
        v[j] = c < nch ? peek(src + c * PCH + 2 + l) : want;
        m[j] = (c < nch && l < 2) ? peek(src + c * PCH + l) : want;
      }
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int c = c0 + 4 * j;
      if (c < nch) {
        dst[c * (DK + 2) + 2 + l] = __uint_as_float(static_cast<uint32_t>(v[j]));
        if (l < 2) dst[c * (DK + 2) + l] = __uint_as_float(static_cast<uint32_t>(m[j]));
      }
    }
  }
}

// This lane's slice of a K-long row: 16-byte pieces (j·64 + lane)·VEC, j < K/(64·VEC).
template <typename T, int K>
struct RowSlice {
  static constexpr int VEC = V16<T>::n;
  static constexpr int J = K / (64 * VEC);
  typename V16<T>::type v[J];
};

template <typename T, int K>
__device__ __forceinline__ void load_row(const T* W, long long row, RowSlice<T, K>& s) {
  const int lane = threadIdx.x & 63;
  const T* p = W + row * K + lane * RowSlice<T, K>::VEC;
#pragma unroll
  for (int j = 0; j < RowSlice<T, K>::J; ++j)
    s.v[j] = *reinterpret_cast<const typename V16<T>::type*>(p + j * 64 * RowSlice<T, K>::VEC);
}

// acc + Σ_e a[e]·b[e] over one 16-byte piece: fp16 pairs on v_dot2_f32_f16 (the two
// products exact in fp32), fp32 by fused multiply-adds.
template <typename T>
__device__ __forceinline__ float dot16(const typename V16<T>::type& a,
                                       const typename V16<T>::type& b, float acc) {
  if constexpr (sizeof(T) == 2) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
#pragma unroll
    for (int e = 0; e < 8; e += 2)
      acc = __builtin_amdgcn_fdot2(h2{a[e], a[e + 1]}, h2{b[e], b[e + 1]}, acc, false);
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) acc += a[e] * b[e];
  }
  return acc;
}

// Lane-partial dot product of a row slice with x (LDS, same slicing); not reduced.
template <typename T, int K>
__device__ __forceinline__ float dot_slice(const RowSlice<T, K>& s, const T* x) {
  const int lane = threadIdx.x & 63;
  constexpr int VEC = RowSlice<T, K>::VEC;
  float acc = 0.f;
#pragma unroll
  for (int j = 0; j < RowSlice<T, K>::J; ++j) {
    const typename V16<T>::type xv =
        *reinterpret_cast<const typename V16<T>::type*>(x + (j * 64 + lane) * VEC);
    acc = dot16<T>(s.v[j], xv, acc);
  }
  return acc;
}

// RMSNorm of the D values in x (LDS), as this lane's slice of the result: lane l of
// every wave holds elements (j·64 + l)·VEC + e, the slice dot_slice multiplies. Each
// wave covers all D elements, so it sums the squares itself (no barrier, no LDS round
// trip) and normalises only what its rows need; g is the same slice of the gain.
// Element arithmetic of kernels/fused_rmsnorm.py:153-162 (fp16: `inv` rounded to fp16)
// and :159-161 (fp32).
template <typename T, int D>
__device__ __forceinline__ void rmsnorm_slice(const T* x, const RowSlice<T, D>& g, RowSlice<T, D>& y) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  constexpr int VEC = RowSlice<T, D>::VEC, J = RowSlice<T, D>::J;
  typename V16<T>::type xv[J];
  float acc = 0.f;
#pragma unroll
  for (int j = 0; j < J; ++j) {
    xv[j] = *reinterpret_cast<const typename V16<T>::type*>(x + (j * 64 + lane) * VEC);
    if constexpr (sizeof(T) == 2) {
      // rnd(v·v) is the fp16 product (packed, two per instruction); pairs of squares are
      // added to the fp32 sum by v_dot2_f32_f16 against (1, 1)
      typedef _Float16 h2 __attribute__((ext_vector_type(2)));
      const typename V16<T>::type sq = xv[j] * xv[j];
      const h2 one2 = {static_cast<_Float16>(1.0f), static_cast<_Float16>(1.0f)};
#pragma unroll
      for (int e = 0; e < VEC; e += 2)
        acc = __builtin_amdgcn_fdot2(h2{sq[e], sq[e + 1]}, one2, acc, false);
    } else {
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const float v = static_cast<float>(xv[j][e]);
        acc += rnd<T>(v * v);
      }
    }
  }
  const float m = wave_sum_dpp(acc) / static_cast<float>(D);
  const float r = sqrtf(m + 1e-5f);
  if constexpr (sizeof(T) == 2) {
    // rnd(rnd(x·inv)·g) with inv rounded to fp16: two fp16 products (packed)
    const T hv = static_cast<T>(rnd<T>(1.0f / r));
    const typename V16<T>::type inv8 = {hv, hv, hv, hv, hv, hv, hv, hv};
#pragma unroll
    for (int j = 0; j < J; ++j) y.v[j] = (xv[j] * inv8) * g.v[j];
  } else {
#pragma unroll
    for (int j = 0; j < J; ++j)
#pragma unroll
      for (int e = 0; e < VEC; ++e)
        y.v[j][e] = static_cast<T>((static_cast<float>(xv[j][e]) / r) * static_cast<float>(g.v[j][e]));
  }
}

// Lane-partial dot product of two row slices (the order of dot_slice); not reduced.
template <typename T, int K>
__device__ __forceinline__ float dot_regs(const RowSlice<T, K>& w, const RowSlice<T, K>& y) {
  float acc = 0.f;
#pragma unroll
  for (int j = 0; j < RowSlice<T, K>::J; ++j) acc = dot16<T>(w.v[j], y.v[j], acc);
  return acc;
}

// Raw 8-element piece (16 B of fp16, 32 B of fp32) and its float values.
template <typename T>
struct Raw8 {
  typename V16<T>::type v[8 / V16<T>::n];
};

template <typename T>
__device__ __forceinline__ void load8(const T* p, Raw8<T>& r) {
#pragma unroll
  for (int i = 0; i < 8 / V16<T>::n; ++i)
    r.v[i] = *reinterpret_cast<const typename V16<T>::type*>(p + i * V16<T>::n);
}

template <typename T>
__device__ __forceinline__ float at8(const Raw8<T>& r, int e) {
  return static_cast<float>(r.v[e / V16<T>::n][e % V16<T>::n]);
}

template <typename T>
__device__ __forceinline__ const T* layer_ptr(const void* base, int l, long long bytes) {
  return reinterpret_cast<const T*>(static_cast<const char*>(base) + l * bytes);
}

// Rows of a phase for this wave: wave w takes local rows w, w+4, …; local rows past
// `R` repeat row 0 (loaded, never stored) so every load is unconditional.
template <int RW>
struct RowSet {
  int row[RW];
  bool live[RW];
};

template <typename T, int D, int DK>
__global__ __launch_bounds__(kT) void decode_persist_kernel(PersistArgs a) {
#pragma clang fp contract(off)
  constexpr int F = 4 * D;
  constexpr int H = D / DK;
  constexpr int TEAM = kG / H;             // workgroups per head (on one XCD)
  constexpr int R_QKV = 3 * DK / TEAM;     // QKV rows per workgroup
  constexpr int R_WO = D / kG;
  constexpr int R_W1 = F / kG;
  constexpr int R_W2 = D / kG;
  constexpr int RW_QKV = (R_QKV + 3) / 4;  // rows per wave
  constexpr int RW_WO = (R_WO + 3) / 4;
  constexpr int RW_W1 = (R_W1 + 3) / 4;
  constexpr int RW_W2 = (R_W2 + 3) / 4;
  constexpr int DG = DK / 8;               // 8-dim groups of a head
  constexpr int NKS = kT / DG;             // key sets in the P·V product
  constexpr int KPT = kChunk / NKS;        // keys per thread in P·V
  constexpr int DPT = DK / 4;              // dims per thread in q·k
  constexpr int NPART = (kMaxCh * (DK + 2) + kT - 1) / kT;
  static_assert(H % kXcd == 0 && kG % H == 0 && (3 * DK) % TEAM == 0, "head teams");
  static_assert(D % kT == 0 && F % kT == 0 && D % kG == 0, "shapes");
  static_assert(R_QKV == 4 * RW_QKV && R_WO == 4 * RW_WO && R_W2 == 4 * RW_W2 && R_W1 == 4 * RW_W1 &&
                    RW_W1 % 2 == 0,
                "every wave owns whole rows (and W1 row pairs) of every phase");
  static_assert(DK % 32 == 0 && DK <= 128 && 3 * DK <= kT, "head dim");

  __shared__ __attribute__((aligned(16))) T s_x[D];   // x of the layer
  __shared__ __attribute__((aligned(16))) T s_xn[D];  // normalised x, or attention output
  __shared__ __attribute__((aligned(16))) T s_xm[D];  // x_mid
  __shared__ __attribute__((aligned(16))) T s_h[F];   // FFN hidden
  __shared__ float s_q[DK], s_kn[DK], s_vn[DK];
  __shared__ float s_o[NKS][DK + 1];
  __shared__ float s_part[NPART * kT];
  __shared__ float s_red[8];
  __shared__ int s_redi[4];

  const int g = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int bad = 0;
  int* err = a.err;
  u64* const slots = a.slots;
  const uint32_t ep = *a.epoch;
  const uint32_t TS = 8u * static_cast<uint32_t>(a.L) + 8u;
  const uint32_t base = ep * TS;
  const int pos = a.pos[0];
  const int len = pos + 1;
  const int nch = (len + kChunk - 1) / kChunk;
  const float scale_t = static_cast<float>(static_cast<T>(a.scale));
  const long long LB = a.layer_bytes;

  // slot regions
  typedef SlotLayout<D, DK> SL;
  u64* X = slots + SL::X;
  u64* QKV = slots + SL::QKV;
  u64* ATT = slots + SL::ATT;
  u64* XM = slots + SL::XM;
  u64* HID = slots + SL::HID;
  u64* PART = slots + SL::PART;
  u64* ARG = slots + SL::ARG;

  // head team of this workgroup
  const int xcd = g % kXcd, kk = g / kXcd;
  const int head = xcd + kXcd * (kk / TEAM);
  const int tm = kk % TEAM;

  const T* emb = static_cast<const T*>(a.emb);
  const T* posw = static_cast<const T*>(a.posw);
  u64* const trace = a.trace ? a.trace + static_cast<long long>(g) * persist_trace_stride(a.L) : nullptr;
  NML_MARK(0);
  if (trace && tid == 0) {  // mark 2: the XCD this workgroup runs on (placement check)
    unsigned xcc;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
    trace[2] = xcc & 0xfu;
  }

  // ---- embedding, computed by every workgroup (no exchange needed)
  {
    const int64_t tok = a.tokens[pos];
    const bool ok = tok >= 0 && tok < a.V && pos >= 0 && pos < a.P;
    if (!ok && tid == 0 && g == 0) atomicOr(err, 1);
    for (int i = tid; i < D; i += kT)
      s_x[i] = ok ? static_cast<T>(static_cast<float>(emb[tok * D + i]) +
                                   static_cast<float>(posw[static_cast<long long>(pos) * D + i]))
                  : static_cast<T>(0.f);
  }
  __syncthreads();
  NML_MARK(1);

  for (int l = 0; l < a.L; ++l) {
    const uint32_t tg = base + 8u * l;
    const int mk = 4 + kMarks * l;
    // ------------------------------------------------------------------ P1
    {
      const T* W = layer_ptr<T>(a.wqkv, l, LB);
      const T* Bq = layer_ptr<T>(a.bqkv, l, LB);
      const T* G1 = layer_ptr<T>(a.ln1, l, LB);
      RowSlice<T, D> w[RW_QKV];
      RowSet<RW_QKV> rs;
      T braw[RW_QKV];
#pragma unroll
      for (int i = 0; i < RW_QKV; ++i) {
        const int rl = wave + 4 * i;
        rs.live[i] = rl < R_QKV;
        const int r = tm * R_QKV + (rs.live[i] ? rl : 0);  // row within the head's 3·DK
        rs.row[i] = (r / DK) * D + head * DK + (r % DK);
        load_row<T, D>(W, rs.row[i], w[i]);
        braw[i] = Bq[rs.row[i]];
      }
      RowSlice<T, D> gsl;
      load_row<T, D>(G1, 0, gsl);
      NML_MARK(mk + 0);
      if (l > 0) {
        gather_lines<T, kG, R_W2, 1, SL::SX>(X, tg, s_x, err, bad);
        __syncthreads();
      }
      NML_MARK(mk + 1);
      RowSlice<T, D> y;
      rmsnorm_slice<T, D>(s_x, gsl, y);
#pragma unroll
      for (int i = 0; i < RW_QKV; ++i) {
        const float acc = wave_sum_dpp(dot_regs<T, D>(w[i], y));
        if (lane == 0 && rs.live[i]) {
          const float lin = rnd<T>(rnd<T>(acc) + static_cast<float>(braw[i]));
          const int r = rs.row[i];
          put(QKV + (head * TEAM + tm) * SL::SQ + wave + 4 * i, tg + 1, enc<T>(lin));
          const int part = r / D, j = r % DK;
          if (part > 0) {
            T* cache = static_cast<T*>(part == 1 ? a.kc : a.vc);
            cache[l * a.kv_layer + head * a.kv_head + static_cast<long long>(pos) * DK + j] =
                static_cast<T>(lin);
          }
        }
      }
      NML_MARK(mk + 2);
    }
    // ------------------------------------------------------------------ P2
    if (tm < nch) {
      const T* Kc = static_cast<const T*>(a.kc) + l * a.kv_layer + head * a.kv_head;
      const T* Vc = static_cast<const T*>(a.vc) + l * a.kv_layer + head * a.kv_head;
      const int qq = tid & 3, dg = tid % DG, ks = tid / DG;
      const bool owns_new = ((nch - 1) % TEAM) == tm;
      bool first = true;
      for (int c = tm; c < nch; c += TEAM) {
        const int k0 = c * kChunk;
        // loads of the chunk (keys clamped into [0, len): stale rows are never used)
        const int key = k0 + (tid >> 2);
        const int keyc = key < len ? key : len - 1;
        Raw8<T> kr[DPT / 8];
#pragma unroll
        for (int e = 0; e < DPT / 8; ++e)
          load8<T>(Kc + static_cast<long long>(keyc) * DK + qq * DPT + e * 8, kr[e]);
        Raw8<T> vr[KPT];
#pragma unroll
        for (int i = 0; i < KPT; ++i) {
          const int vk = k0 + 16 * wave + (lane >> 3) + 8 * i;
          load8<T>(Vc + static_cast<long long>(vk < len ? vk : len - 1) * DK + dg * 8, vr[i]);
        }
        if (first) {  // q, and k/v of the new position for the workgroup that owns it
          NML_MARK(mk + 14);
          int idx[1];
          uint32_t pv[1];
          const int part = tid / DK, j = tid % DK;  // tid = row within the head's 3·DK
          idx[0] = (tid < DK || (owns_new && tid < 3 * DK))
                       ? (head * TEAM + tid / R_QKV) * SL::SQ + tid % R_QKV
                       : -1;
          wait_slots<1>(QKV, idx, tg + 1, pv, err, bad);
          if (idx[0] >= 0) (part == 0 ? s_q : part == 1 ? s_kn : s_vn)[j] = static_cast<float>(dec<T>(pv[0]));
          first = false;
          __syncthreads();
          NML_MARK(mk + 3);
        }
        const bool kvalid = key < len;
        float dot = 0.f;
        if (key == pos) {
#pragma unroll
          for (int e = 0; e < DPT; ++e) dot += s_q[qq * DPT + e] * s_kn[qq * DPT + e];
        } else {
#pragma unroll
          for (int e = 0; e < DPT; ++e) dot += s_q[qq * DPT + e] * at8<T>(kr[e / 8], e % 8);
        }
        dot = quad_sum_dpp(dot);
        // Each wave takes the softmax of its own 16 keys against its own maximum; the
        // waves' (max, sum, P·V) are combined after one barrier below.
        const float sc = kvalid ? rnd<T>(rnd<T>(dot) / scale_t) : -INFINITY;
        const float mw = wave_max_dpp(sc);
        const float p = kvalid ? expf(sc - mw) : 0.f;
        const float lw = wave_sum_dpp(qq == 0 ? p : 0.f);
        float o[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = 0.f;
#pragma unroll
        for (int i = 0; i < KPT; ++i) {
          const int jj = (lane >> 3) + 8 * i, vk = k0 + 16 * wave + jj;  // key jj of the wave's 16
          const float pj = __shfl(p, 4 * jj, 64);
          // Row `pos` of the cache may not be written yet in this step (and clamped
          // keys past len read it): those keys never touch the loaded values.
          if (vk == pos) {
#pragma unroll
            for (int e = 0; e < 8; ++e) o[e] += pj * s_vn[dg * 8 + e];
          } else if (vk < len) {
#pragma unroll
            for (int e = 0; e < 8; ++e) o[e] += pj * at8<T>(vr[i], e);
          }
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) s_o[ks][dg * 8 + e] = o[e];
        if (lane == 0) {
          s_red[wave] = mw;
          s_red[4 + wave] = lw;
        }
        __syncthreads();
        u64* dst = PART + (static_cast<long long>(head) * kMaxCh + c) * SL::PCH;
        if (tid <= DK) {
          const float M = fmaxf(fmaxf(s_red[0], s_red[1]), fmaxf(s_red[2], s_red[3]));
          float f[4];
#pragma unroll
          for (int w2 = 0; w2 < 4; ++w2) f[w2] = s_red[w2] == -INFINITY ? 0.f : expf(s_red[w2] - M);
          if (tid < DK) {
            float s = 0.f;
#pragma unroll
            for (int w2 = 0; w2 < 4; ++w2) {
              float sw = 0.f;
#pragma unroll
              for (int k2 = 0; k2 < NKS / 4; ++k2) sw += s_o[w2 * (NKS / 4) + k2][tid];
              s += f[w2] * sw;
            }
            put(dst + 2 + tid, tg + 2, __float_as_uint(s));
          } else {
            const float L = (f[0] * s_red[4] + f[1] * s_red[5]) + (f[2] * s_red[6] + f[3] * s_red[7]);
            put(dst, tg + 2, __float_as_uint(M));
            put(dst + 1, tg + 2, __float_as_uint(L));
          }
        }
        __syncthreads();
      }
      NML_MARK(mk + 4);
    }
    // ------------------------------------------------------------------ P2b
    if (tm == 0) {
      gather_partials<DK, SL::PCH>(PART + static_cast<long long>(head) * kMaxCh * SL::PCH, nch,
                                   tg + 2, s_part, err, bad);
      __syncthreads();
      if (tid < DK) {  // wave 0: lane c holds chunk c's (max, sum), lane d sums dim d
        static_assert(kMaxCh <= 64, "one lane per chunk");
        const bool has = lane < nch;
        const float mcl = has ? s_part[lane * (DK + 2)] : -INFINITY;
        const float M = wave_max_dpp(mcl);
        const float ec = has ? expf(mcl - M) : 0.f;
        const float den = wave_sum_dpp(has ? ec * s_part[lane * (DK + 2) + 1] : 0.f);
        float num = 0.f;
        for (int c = 0; c < nch; ++c) num += lane_f(ec, c) * s_part[c * (DK + 2) + 2 + tid];
        const float o = num * (1.f / den);
        const float o1 = __shfl_xor(o, 1, 64);  // dims 2k, 2k+1 share a slot
        if ((tid & 1) == 0) put_pair<T>(ATT + head * (DK / kPack<T>), tid, tg + 3, o, o1);
      }
      NML_MARK(mk + 5);
    }
    // ------------------------------------------------------------------ P3
    {
      const T* W = layer_ptr<T>(a.wo, l, LB);
      const T* Bo = layer_ptr<T>(a.bo, l, LB);
      RowSlice<T, D> w[RW_WO];
      RowSet<RW_WO> rs;
      T braw[RW_WO];
#pragma unroll
      for (int i = 0; i < RW_WO; ++i) {
        const int rl = wave + 4 * i;
        rs.live[i] = rl < R_WO;
        rs.row[i] = g * R_WO + (rs.live[i] ? rl : 0);
        load_row<T, D>(W, rs.row[i], w[i]);
        braw[i] = Bo[rs.row[i]];
      }
      NML_MARK(mk + 15);
      gather<T, D, kPack<T>>(ATT, tg + 3, s_xn, err, bad);
      __syncthreads();
      NML_MARK(mk + 6);
#pragma unroll
      for (int i = 0; i < RW_WO; ++i) {
        const float acc = wave_sum_dpp(dot_slice<T, D>(w[i], s_xn));
        if (lane == 0 && rs.live[i]) {
          const float lin = rnd<T>(rnd<T>(acc) + static_cast<float>(braw[i]));
          put(XM + g * SL::SX + wave + 4 * i, tg + 4,
              enc<T>(static_cast<float>(s_x[rs.row[i]]) + lin));
        }
      }
      NML_MARK(mk + 10);
    }
    // ------------------------------------------------------------------ P4
    {
      const T* W = layer_ptr<T>(a.w1, l, LB);
      const T* B1 = layer_ptr<T>(a.b1, l, LB);
      const T* G2 = layer_ptr<T>(a.ln2, l, LB);
      RowSlice<T, D> w[RW_W1];
      RowSet<RW_W1> rs;
      T braw[RW_W1];
      // row pairs (2k, 2k+1), k = wave, wave+4, …: one slot of h carries both
#pragma unroll
      for (int i = 0; i < RW_W1; ++i) {
        rs.live[i] = true;
        rs.row[i] = g * R_W1 + 2 * (wave + 4 * (i >> 1)) + (i & 1);
        load_row<T, D>(W, rs.row[i], w[i]);
        braw[i] = B1[rs.row[i]];
      }
      RowSlice<T, D> gsl;
      load_row<T, D>(G2, 0, gsl);
      NML_MARK(mk + 11);
      gather_lines<T, kG, R_WO, 1, SL::SX>(XM, tg + 4, s_xm, err, bad);
      __syncthreads();
      NML_MARK(mk + 7);
      RowSlice<T, D> y;
      rmsnorm_slice<T, D>(s_xm, gsl, y);
#pragma unroll
      for (int i = 0; i < RW_W1; i += 2) {
        float v[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const float acc = wave_sum_dpp(dot_regs<T, D>(w[i + h], y));
          v[h] = gelu_t<T>(rnd<T>(rnd<T>(acc) + static_cast<float>(braw[i + h])));
        }
        if (lane == 0) put_pair<T>(HID + g * SL::SH, rs.row[i] - g * R_W1, tg + 5, v[0], v[1]);
      }
      NML_MARK(mk + 12);
    }
    // ------------------------------------------------------------------ P5
    {
      const T* W = layer_ptr<T>(a.w2, l, LB);
      const T* B2 = layer_ptr<T>(a.b2, l, LB);
      RowSlice<T, F> w[RW_W2];
      RowSet<RW_W2> rs;
      T braw[RW_W2];
#pragma unroll
      for (int i = 0; i < RW_W2; ++i) {
        const int rl = wave + 4 * i;
        rs.live[i] = rl < R_W2;
        rs.row[i] = g * R_W2 + (rs.live[i] ? rl : 0);
        load_row<T, F>(W, rs.row[i], w[i]);
        braw[i] = B2[rs.row[i]];
      }
      NML_MARK(mk + 13);
      gather_lines<T, kG, R_W1, kPack<T>, SL::SH>(HID, tg + 5, s_h, err, bad);
      __syncthreads();
      NML_MARK(mk + 8);
#pragma unroll
      for (int i = 0; i < RW_W2; ++i) {
        const float acc = wave_sum_dpp(dot_slice<T, F>(w[i], s_h));
        if (lane == 0 && rs.live[i]) {
          const float lin = rnd<T>(rnd<T>(acc) + static_cast<float>(braw[i]));
          put(X + g * SL::SX + wave + 4 * i, tg + 8,
              enc<T>(static_cast<float>(s_xm[rs.row[i]]) + lin));
        }
      }
      NML_MARK(mk + 9);
    }
  }
  const int mh = 4 + kMarks * a.L;

  // ---------------------------------------------------------------- head
  const uint32_t tgh = base + 8u * a.L;
  constexpr int HR = 8;  // rows per wave per round
  const int r0 = static_cast<int>((static_cast<long long>(g) * a.V) / kG);
  const int r1 = static_cast<int>((static_cast<long long>(g + 1) * a.V) / kG);
  const T* E = emb;
  RowSlice<T, D> cur[HR];
  int rb = r0 + wave * HR;
#pragma unroll
  for (int i = 0; i < HR; ++i) load_row<T, D>(E, rb + i < r1 ? rb + i : r0, cur[i]);
  RowSlice<T, D> y;
  {
    RowSlice<T, D> gsl;
    load_row<T, D>(static_cast<const T*>(a.lnf), 0, gsl);
    gather_lines<T, kG, R_W2, 1, SL::SX>(X, tgh, s_x, err, bad);
    __syncthreads();
    NML_MARK(mh + 0);
    rmsnorm_slice<T, D>(s_x, gsl, y);
  }
  T* logits = static_cast<T*>(a.logits);
  float best = -INFINITY;
  int bi = 0x7fffffff;
  for (; rb < r1; rb += 4 * HR) {
    RowSlice<T, D> nxt[HR];
    const int rn = rb + 4 * HR;
#pragma unroll
    for (int i = 0; i < HR; ++i) load_row<T, D>(E, rn + i < r1 ? rn + i : r0, nxt[i]);
#pragma unroll
    for (int i = 0; i < HR; ++i) {
      const float acc = wave_sum_dpp(dot_regs<T, D>(cur[i], y));
      const float v = rnd<T>(acc);
      if (rb + i < r1) {
        if (lane == 0) logits[rb + i] = static_cast<T>(v);
        if (v > best || (v == best && rb + i < bi)) {
          best = v;
          bi = rb + i;
        }
      }
    }
#pragma unroll
    for (int i = 0; i < HR; ++i) cur[i] = nxt[i];
  }
  NML_MARK(mh + 1);
  if (lane == 0) {
    s_red[wave] = best;
    s_redi[wave] = bi;
  }
  __syncthreads();
  if (tid == 0) {
    float bb = s_red[0];
    int ii = s_redi[0];
    for (int w2 = 1; w2 < 4; ++w2)
      if (s_red[w2] > bb || (s_red[w2] == bb && s_redi[w2] < ii)) {
        bb = s_red[w2];
        ii = s_redi[w2];
      }
    put(ARG + g * kLine, tgh + 1, __float_as_uint(bb));
    put(ARG + g * kLine + 1, tgh + 1, static_cast<uint32_t>(ii));
  }
  if (g == 0) {
    __syncthreads();
    int idx[2] = {tid < kG ? tid * kLine : -1, tid < kG ? tid * kLine + 1 : -1};
    uint32_t pv[2];
    wait_slots<2>(ARG, idx, tgh + 1, pv, err, bad);
    float b = tid < kG ? __uint_as_float(pv[0]) : -INFINITY;
    int i = tid < kG ? static_cast<int>(pv[1]) : 0x7fffffff;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const float ob = __shfl_xor(b, o, 64);
      const int oi = __shfl_xor(i, o, 64);
      if (ob > b || (ob == b && oi < i)) {
        b = ob;
        i = oi;
      }
    }
    if (lane == 0) {
      s_red[wave] = b;
      s_redi[wave] = i;
    }
    __syncthreads();
    if (tid == 0) {
      float bb = s_red[0];
      int ii = s_redi[0];
      for (int w2 = 1; w2 < 4; ++w2)
        if (s_red[w2] > bb || (s_red[w2] == bb && s_redi[w2] < ii)) {
          bb = s_red[w2];
          ii = s_redi[w2];
        }
      if (a.fuse_argmax) {
        a.tokens[pos + 1] = ii;
        a.pos[0] = pos + 1;
      }
      *a.epoch = ep + 1;
      NML_MARK(mh + 2);
    }
  }
}

template <typename T, int D, int DK>
int launch_typed(const PersistArgs& a, hipStream_t st) {
  decode_persist_kernel<T, D, DK><<<kG, kT, 0, st>>>(a);
  NML_LAUNCHED();
  return 0;
}

}  // namespace

bool persist_supported(int dt, int d, int H, int F, int B, int P) {
  if (B != 1 || F != 4 * d || P > kPersistMaxLen || H <= 0 || d % H != 0) return false;
  const int dk = d / H;
  if (dk != 64 || d != 1024 || (dt != F16 && dt != F32)) return false;
  // All kG workgroups must be resident at once: they wait on each other.
  static int resident[2] = {-1, -1};
  int& r = resident[dt == F16 ? 1 : 0];
  if (r < 0) {
    int dev = 0, per_cu = 0;
    hipDeviceProp_t prop;
    r = 0;
    if (hipGetDevice(&dev) == hipSuccess && hipGetDeviceProperties(&prop, dev) == hipSuccess) {
      const void* fn = dt == F16 ? reinterpret_cast<const void*>(&decode_persist_kernel<half_t, 1024, 64>)
                                 : reinterpret_cast<const void*>(&decode_persist_kernel<float, 1024, 64>);
      if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, kT, 0) == hipSuccess)
        r = per_cu * prop.multiProcessorCount >= kG ? 1 : 0;
    }
  }
  return r == 1;
}

size_t persist_slot_count(int d, int H) {
  // the persistent kernel exists for d = 1024, head dim 64 only (persist_supported)
  (void)d;
  (void)H;
  return SlotLayout<1024, 64>::total;
}

int launch_decode_persist(int dt, int d, int H, const PersistArgs& a, hipStream_t st) {
  const int dk = d / H;
  NML_REQUIRE(a.pos != nullptr && a.tokens != nullptr && a.slots != nullptr && a.epoch != nullptr,
              "persistent decode: state pointers missing");
  if (dt == F16 && d == 1024 && dk == 64) return launch_typed<half_t, 1024, 64>(a, st);
  if (dt == F32 && d == 1024 && dk == 64) return launch_typed<float, 1024, 64>(a, st);
  set_error("persistent decode: unsupported shape d=%d dk=%d dtype=%d", d, dk, dt);
  return -1;
}

}  // namespace nml
