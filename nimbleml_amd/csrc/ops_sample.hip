// Next-token selection on device, one 1024-lane workgroup per sequence, following
// _sample_logits (models/generate.py:23-59) step by step:
//   x = float32(logits); repetition penalty on tokens already in the row
//   (generate.py:9-20: x<0 → x·p, else x/p, once per distinct token);
//   T ≤ 0 → argmax (first index on ties);
//   x /= T; top-k keeps x ≥ (k-th largest x) (ties kept, :43-46), others → −1e9;
//   p = exp(x − max) / Σ;
//   no top-p: the token is the first index i (index order) whose float64
//   cumulative p, divided by the total, exceeds u — what RandomState.choice does
//   with its uniform draw u (float64 cumsum, cdf/cdf[-1], searchsorted 'right');
//   top-p (:49-58): walk p in descending order, keep the prefix whose running sum
//   stays ≤ top_p (at least one), renormalise, and pick the first position of
//   that descending order whose float64 running sum / total exceeds u.
// No sort is formed: every "k-th largest" and "first descending position whose
// running mass exceeds a target" is found by a 4-pass, 8-bit radix select over
// the order-preserving integer image of x, with per-bin counts and masses. The
// descending order is the reference's argsort(probs)[::-1]: equal probabilities
// come in descending index order, which is what reversing a stable ascending sort
// gives (NumPy's default argsort is not stable, so the order of exact ties is
// whatever its sort produced; descending index is the stable reading).
// The sampled-decode case (fp16 rows, top-k ≤ 256 without top-p) first tries
// sample_topk_regs: the row stays in registers, and the k-th largest is counted among
// the few elements above a per-wave lower bound; the general path below runs when it
// declines.
#include "kernels.hpp"

namespace nml {

namespace {

constexpr int kThreads = 1024;
constexpr int kWaves = kThreads / 64;
constexpr int kBitmapWords = 2048;  // repetition-penalty membership, V ≤ 65536

__device__ __forceinline__ uint32_t fkey(float f) {
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

struct Shared {
  int hist_cnt[256];
  double hist_mass[256];
  uint32_t bitmap[kBitmapWords];
  float redf[kWaves];
  int redi[kWaves];
  double redd[kWaves];
  uint32_t sel_prefix;
  int sel_k;
  double sel_cum;
  int sel_bin_cnt;
  double sel_bin_mass;
  int found_index;
  float reg_thr, reg_max;  // sample_topk_regs: the k-th largest s and the largest
};

__device__ float block_max_f(float v, Shared& sh) {
  v = wave_max(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) sh.redf[threadIdx.x >> 6] = v;
  __syncthreads();
  float t = sh.redf[0];
  for (int i = 1; i < kWaves; ++i) t = fmaxf(t, sh.redf[i]);
  return t;
}

__device__ float block_sum_f(float v, Shared& sh) {
  v = wave_sum(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) sh.redf[threadIdx.x >> 6] = v;
  __syncthreads();
  float t = 0.f;
  for (int i = 0; i < kWaves; ++i) t += sh.redf[i];
  return t;
}

// Exclusive prefix over threads (thread order) of a double; also returns the total.
__device__ double block_excl_scan_d(double v, double* total, Shared& sh) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  double inc = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const double t = __shfl_up(inc, o, 64);
    if (lane >= o) inc += t;
  }
  __syncthreads();
  if (lane == 63) sh.redd[w] = inc;
  __syncthreads();
  double before = 0.0, tot = 0.0;
  for (int i = 0; i < kWaves; ++i) {
    if (i < w) before += sh.redd[i];
    tot += sh.redd[i];
  }
  *total = tot;
  return before + inc - v;
}

__device__ int block_excl_scan_i(int v, int* total, Shared& sh) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  int inc = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int t = __shfl_up(inc, o, 64);
    if (lane >= o) inc += t;
  }
  __syncthreads();
  if (lane == 63) sh.redi[w] = inc;
  __syncthreads();
  int before = 0, tot = 0;
  for (int i = 0; i < kWaves; ++i) {
    if (i < w) before += sh.redi[i];
    tot += sh.redi[i];
  }
  *total = tot;
  return before + inc - v;
}

template <typename T>
struct Row {
  const T* lg;
  int V;
  float pen;
  float inv_t;       // unused when greedy
  float temperature;
  bool use_pen;
  const uint32_t* bitmap;

  // Penalised float32 logit (generate.py:34-37 then :9-20) of the value x at index i.
  __device__ float penalised(float x, int i) const {
    if (use_pen && ((bitmap[i >> 5] >> (i & 31)) & 1u)) x = x < 0.f ? x * pen : x / pen;
    return x;
  }
  __device__ float base(int i) const { return penalised(static_cast<float>(lg[i]), i); }
  // After temperature (generate.py:42): float32 division by float32(T).
  __device__ float scaled(int i) const { return base(i) / temperature; }
};

// k-th largest key among keys of x over all i (k ≥ 1).
template <typename F>
__device__ uint32_t select_kth_key(int V, int k, F key_of, Shared& sh) {
  uint32_t prefix = 0, mask = 0;
  if (threadIdx.x == 0) sh.sel_k = k;
  for (int shift = 24; shift >= 0; shift -= 8) {
    for (int i = threadIdx.x; i < 256; i += kThreads) sh.hist_cnt[i] = 0;
    __syncthreads();
    for (int i = threadIdx.x; i < V; i += kThreads) {
      const uint32_t key = key_of(i);
      if ((key & mask) == prefix) atomicAdd(&sh.hist_cnt[(key >> shift) & 255u], 1);
    }
    __syncthreads();
    if (threadIdx.x < 64) {
      // wave 0: lane l owns bins 255-4l … 252-4l (descending); an exclusive prefix of
      // the lanes' counts finds the bin holding the k-th largest key
      const int l = threadIdx.x, kk = sh.sel_k;
      int c4[4], own = 0;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        c4[e] = sh.hist_cnt[255 - 4 * l - e];
        own += c4[e];
      }
      int inc = own;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int t = __shfl_up(inc, o, 64);
        if (l >= o) inc += t;
      }
      int cum = inc - own;
      if (cum < kk && inc >= kk) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if (cum + c4[e] >= kk) {
            sh.sel_k = kk - cum;
            sh.sel_prefix = prefix | (static_cast<uint32_t>(255 - 4 * l - e) << shift);
            break;
          }
          cum += c4[e];
        }
      }
    }
    __syncthreads();
    prefix = sh.sel_prefix;
    mask |= 255u << shift;
  }
  return prefix;
}

// Most candidates (elements ≥ a top-k threshold or its lower bound) held in LDS.
constexpr int kCandMax = 2048;

// Wave 0 draws over n candidates (index order, candx = scaled logits) keeping those
// ≥ thresh: max, Σ exp, probabilities and the float64 index-order CDF; returns the first
// kept index whose cdf / total exceeds u (the last kept index if rounding leaves none,
// where the reference's cdf / cdf[-1] is exactly 1). All threads must call it (barriers).
template <typename T>
__device__ int draw_candidates(int V, int n, float thresh, double u, Shared& sh, const int* cand,
                               const float* candx) {
  if (threadIdx.x < 64) {
    const int l = threadIdx.x;
    float mx = -INFINITY;
    for (int j = l; j < n; j += 64)
      if (candx[j] >= thresh) mx = fmaxf(mx, candx[j]);
    mx = wave_max(mx);
    float se = 0.f;
    for (int j = l; j < n; j += 64)
      if (candx[j] >= thresh) se += expf(candx[j] - mx);
    se = wave_sum(se);
    double total = 0.0;
    for (int j = l; j < n; j += 64)
      if (candx[j] >= thresh) total += static_cast<double>(expf(candx[j] - mx) / se);
    total = wave_sum_d(total);
    // index-order running sums, 64 candidates per round
    double carry = 0.0;
    int found = 0x7fffffff, last_kept = V - 1;
    for (int j0 = 0; j0 < n && found == 0x7fffffff; j0 += 64) {
      const int j = j0 + l;
      const bool keep = j < n && candx[j] >= thresh;
      const double pj = keep ? static_cast<double>(expf(candx[j] - mx) / se) : 0.0;
      double inc = pj;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const double t = __shfl_up(inc, o, 64);
        if (l >= o) inc += t;
      }
      const bool hit = keep && (carry + inc) / total > u;
      const unsigned long long hits = __ballot(hit);
      const unsigned long long kept = __ballot(keep);
      if (hits) found = cand[j0 + __ffsll(static_cast<long long>(hits)) - 1];
      if (kept) last_kept = cand[j0 + 63 - __clzll(static_cast<long long>(kept))];
      carry += __shfl(inc, 63, 64);
    }
    // none hit (the scan's running sum ends an ulp below `total`): the reference's
    // searchsorted over cdf / cdf[-1] lands on the last kept index, where that ratio is 1
    if (l == 0) sh.found_index = found == 0x7fffffff ? last_kept : found;
  }
  __syncthreads();
  return sh.found_index;
}

// Gather the elements with scaled logit ≥ lo into cand / candx in index order; returns
// their count, or -1 if more than kCandMax.
template <typename T>
__device__ int gather_candidates(const Row<T>& row, float lo, Shared& sh, int* cand, float* candx) {
  const int V = row.V;
  const int seg = (V + kThreads - 1) / kThreads;
  const int b0 = threadIdx.x * seg, b1 = min(V, b0 + seg);
  int c = 0;
  for (int i = b0; i < b1; ++i) c += row.scaled(i) >= lo ? 1 : 0;
  int n = 0;
  int off = block_excl_scan_i(c, &n, sh);
  if (n > kCandMax) return -1;
  for (int i = b0; i < b1; ++i) {
    const float x = row.scaled(i);
    if (x >= lo) {
      cand[off] = i;
      candx[off] = x;
      ++off;
    }
  }
  __syncthreads();
  return n;
}

// Top-k sampling without top-p on fp16 logits held in registers (no LDS copy of the
// row) — the sampled-decode case: 1 ≤ k ≤ kRegK, V a multiple of 8 up to 32·1024,
// 16-byte aligned rows. Thread t holds elements 32t … 32t+31 as penalised float32
// values y; the temperature-scaled value is s = y / T (float32 division), a
// non-decreasing function of y, so every order question is answered on y and s is
// formed only for the elements that can be kept. Every element below the k-th largest
// s becomes -1e9, whose exp(x − max) is exactly 0, so only the elements ≥ it carry mass.
//   1. A lower bound without a block-wide select: each of the nw waves whose lanes all
//      hold elements takes the q-th largest of its 64 lane maxima of y (q = ⌈k / nw⌉)
//      by repeated wave maxima; the smallest of those, L, has ≥ nw·q ≥ k elements
//      at or above it, so the k-th largest s is ≥ L / T.
//   2. y* = the smallest float with y* / T ≥ L / T (a few steps down from L): the
//      elements with y ≥ y* are exactly those with s ≥ L / T, a superset of the kept
//      ones. They are gathered into LDS with s, in index order (threads own
//      consecutive elements).
//   3. Among them, the k-th largest s (#(> s) < k ≤ #(≥ s)) and the maximum by counting.
//   4. draw_kept: the index-order float64 CDF over the kept ones (s ≥ the k-th largest).
// Returns the chosen index, or -1 (the general path then runs) when more than kRegCand
// elements reach y*, or when fewer than k/64 waves are full. All threads must call it.
constexpr int kRegElems = 32;   // elements per thread: V ≤ 32768
constexpr int kRegK = 256;
constexpr int kRegCand = 1024;  // gathered candidates (≤ kCandMax)

__device__ bool sample_regs_applies(const Row<half_t>& row, int k) {
  const int V = row.V;
  return k >= 1 && k <= kRegK && (V & 7) == 0 && V <= kRegElems * kThreads &&
         (reinterpret_cast<uintptr_t>(row.lg) & 15) == 0;
}

__device__ __forceinline__ float prev_float(float y) {
  if (y == 0.f) return -__int_as_float(1);
  const int b = __float_as_int(y);
  return __int_as_float(y > 0.f ? b - 1 : b + 1);
}

// Wave 0 draws over the n candidates (index order; candx = scaled values) keeping those
// ≥ thr, with max mx: p = exp(x − mx) / Σ exp (float32), then the first kept index whose
// float64 running sum / total exceeds u (the last kept index if rounding leaves none).
// n ≤ 64·R.
template <int R>
__device__ __forceinline__ int draw_kept(int V, int n, float thr, float mx, double u, Shared& sh, const int* cand,
                         const float* candx) {
  if (threadIdx.x < 64) {
    const int l = threadIdx.x;
    float e[R];
    float se = 0.f;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int j = l + 64 * r;
      const float x = j < n ? candx[j] : -INFINITY;
      e[r] = x >= thr ? expf(x - mx) : 0.f;
      se += e[r];
    }
    se = wave_sum(se);
    double p[R], total = 0.0;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      p[r] = static_cast<double>(e[r] / se);
      total += p[r];
    }
    total = wave_sum_d(total);
    double carry = 0.0;
    int found = 0x7fffffff, last_kept = V - 1;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if (found != 0x7fffffff || 64 * r >= n) break;
      const int j = l + 64 * r;
      const bool keep = j < n && candx[j] >= thr;
      double inc = p[r];
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const double t = __shfl_up(inc, o, 64);
        if (l >= o) inc += t;
      }
      const unsigned long long hits = __ballot(keep && (carry + inc) / total > u);
      const unsigned long long kept = __ballot(keep);
      if (hits) found = cand[64 * r + __ffsll(static_cast<long long>(hits)) - 1];
      if (kept) last_kept = cand[64 * r + 63 - __clzll(static_cast<long long>(kept))];
      carry += __shfl(inc, 63, 64);
    }
    // none hit: the last kept index, as the reference's searchsorted over cdf / cdf[-1]
    if (l == 0) sh.found_index = found == 0x7fffffff ? last_kept : found;
  }
  __syncthreads();
  return sh.found_index;
}

__device__ __forceinline__ int sample_topk_regs(const Row<half_t> row, int k, double u, Shared& sh,
                                                int* cand, float* candx) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int V = row.V;
  // waves 0 … nw-1 have every lane holding elements (lane 63 of wave w starts at
  // 32·(64w + 63))
  const int last = (V - 1) / kRegElems;  // the last thread holding elements
  const int nw = last < 63 ? 0 : ((last - 63) / 64 + 1 < kWaves ? (last - 63) / 64 + 1 : kWaves);
  if (nw == 0 || (k + nw - 1) / nw > 64) return -1;
  const int q = (k + nw - 1) / nw;
  const int i0 = kRegElems * tid;
  float y[kRegElems];
  float tmax = -INFINITY;
#pragma unroll
  for (int c = 0; c < kRegElems / 8; ++c) {
    if (i0 + 8 * c < V) {
      const half8 h = *reinterpret_cast<const half8*>(row.lg + i0 + 8 * c);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        y[8 * c + e] = row.penalised(static_cast<float>(h[e]), i0 + 8 * c + e);
        tmax = fmaxf(tmax, y[8 * c + e]);
      }
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) y[8 * c + e] = -INFINITY;
    }
  }
  if (wave < nw) {
    // q-th largest lane maximum: each round takes the wave maximum and retires the lanes
    // holding it; the round where the retired count reaches q has it (≤ q rounds)
    float cur = tmax, qv = -INFINITY;
    int rem = q;
    for (int r = 0; r < q; ++r) {
      const float mw = wave_max_dpp(cur);
      const int cnt = __popcll(__ballot(cur == mw));
      if (cnt >= rem) {
        qv = mw;
        break;
      }
      rem -= cnt;
      if (cur == mw) cur = -INFINITY;
    }
    if (lane == 0) sh.redf[wave] = qv;
  }
  __syncthreads();
  // every thread forms the same y* (no broadcast round); INFINITY: give up (n = 0 → -1)
  float lo = INFINITY;
  for (int w = 0; w < nw; ++w) lo = fminf(lo, sh.redf[w]);
  {
    const float ls = lo / row.temperature;
    int steps = 0;
    for (; steps < 64; ++steps) {
      const float yd = prev_float(lo);
      if (!(yd / row.temperature >= ls)) break;
      lo = yd;
    }
    if (steps == 64) lo = INFINITY;
  }
  int c = 0;
#pragma unroll
  for (int j = 0; j < kRegElems; ++j) c += y[j] >= lo ? 1 : 0;
  int inc = c;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int t = __shfl_up(inc, o, 64);
    if (lane >= o) inc += t;
  }
  if (lane == 63) sh.redi[wave] = inc;
  __syncthreads();
  int off = inc - c, n = 0;
  for (int w = 0; w < kWaves; ++w) {
    const int cw = sh.redi[w];
    if (w < wave) off += cw;
    n += cw;
  }
  if (n > kRegCand || n < k) return -1;  // the same n in every thread
#pragma unroll
  for (int j = 0; j < kRegElems; ++j)
    if (y[j] >= lo) {
      cand[off] = i0 + j;
      candx[off] = y[j] / row.temperature;
      ++off;
    }
  const int n4 = (n + 3) & ~3;  // padded to whole float4 reads: -inf never counts
  if (tid >= n && tid < n4) candx[tid] = -INFINITY;
  __syncthreads();
  const float4* cx4 = reinterpret_cast<const float4*>(candx);
  if (tid < n) {  // every thread whose value is the k-th largest writes the same
    const float xt = candx[tid];
    int gt = 0, ge = 0;
    int r = 0;
    for (; r + 4 <= n4 / 4; r += 4) {
      float4 v[4];
#pragma unroll
      for (int h = 0; h < 4; ++h) v[h] = cx4[r + h];
#pragma unroll
      for (int h = 0; h < 4; ++h) {
        gt += (v[h].x > xt) + (v[h].y > xt) + (v[h].z > xt) + (v[h].w > xt);
        ge += (v[h].x >= xt) + (v[h].y >= xt) + (v[h].z >= xt) + (v[h].w >= xt);
      }
    }
    for (; r < n4 / 4; ++r) {
      const float4 v = cx4[r];
      gt += (v.x > xt) + (v.y > xt) + (v.z > xt) + (v.w > xt);
      ge += (v.x >= xt) + (v.y >= xt) + (v.z >= xt) + (v.w >= xt);
    }
    if (gt < k && ge >= k) sh.reg_thr = xt;
    if (gt == 0) sh.reg_max = xt;
  }
  __syncthreads();
  return draw_kept<kRegCand / 64>(row.V, n, sh.reg_thr, sh.reg_max, u, sh, cand, candx);
}

// Top-k sampling without top-p (generate.py:43-47, then RandomState.choice): every
// element below the k-th largest scaled logit T becomes -1e9, whose exp(x − max)
// underflows to exactly 0, so only the elements ≥ T carry mass. T is found without a
// pass over the whole row per radix digit: the k-th largest of the 1024 per-thread
// maxima is a lower bound L ≤ T (at most k threads can hold an element ≥ T), the
// elements ≥ L are gathered (all of the top k among them), and T is selected among
// those. Returns the chosen index, or -1 (k > 1024 or too many candidates: the caller
// runs the full scan).
template <typename T>
__device__ int sample_topk_fast(const Row<T>& row, int k, double u, Shared& sh, int* cand,
                                float* candx, uint32_t* tkeys) {
  const int V = row.V;
  if (k > kThreads) return -1;
  float tm = -INFINITY;
  for (int i = threadIdx.x; i < V; i += kThreads) tm = fmaxf(tm, row.scaled(i));
  tkeys[threadIdx.x] = fkey(tm);
  __syncthreads();
  const uint32_t lk = select_kth_key(kThreads, k, [&](int i) { return tkeys[i]; }, sh);
  const float lo = __uint_as_float((lk & 0x80000000u) ? (lk & 0x7fffffffu) : ~lk);
  const int n = gather_candidates(row, lo, sh, cand, candx);
  if (n < 0) return -1;
  const uint32_t tk = select_kth_key(n, k, [&](int j) { return fkey(candx[j]); }, sh);
  const float thresh = __uint_as_float((tk & 0x80000000u) ? (tk & 0x7fffffffu) : ~tk);
  return draw_candidates<T>(V, n, thresh, u, sh, cand, candx);
}

// The same draw with T already known (the full-scan path): gathers the elements ≥ T.
template <typename T>
__device__ int sample_topk_candidates(const Row<T>& row, float thresh, double u, Shared& sh,
                                      int* cand, float* candx) {
  const int n = gather_candidates(row, thresh, sh, cand, candx);
  if (n < 0) return -1;
  return draw_candidates<T>(row.V, n, thresh, u, sh, cand, candx);
}

// First position of the descending order (key desc, then index desc) over the
// elements with in_set(i) whose inclusive running mass (weights w, equal for equal
// keys) exceeds `target`. Returns the key τ and the 1-based rank of that element
// among the in-set elements with key τ counted in ascending index order.
template <typename FK, typename FW, typename FS>
__device__ void select_by_mass(int V, double target, FK key_of, FW weight, FS in_set,
                               uint32_t* tau, int* rank, Shared& sh) {
  uint32_t prefix = 0, mask = 0;
  if (threadIdx.x == 0) sh.sel_cum = 0.0;
  for (int shift = 24; shift >= 0; shift -= 8) {
    for (int i = threadIdx.x; i < 256; i += kThreads) {
      sh.hist_cnt[i] = 0;
      sh.hist_mass[i] = 0.0;
    }
    __syncthreads();
    for (int i = threadIdx.x; i < V; i += kThreads) {
      if (!in_set(i)) continue;
      const uint32_t key = key_of(i);
      if ((key & mask) == prefix) {
        const uint32_t bin = (key >> shift) & 255u;
        atomicAdd(&sh.hist_cnt[bin], 1);
        atomicAdd(&sh.hist_mass[bin], static_cast<double>(weight(i)));
      }
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      double cum = sh.sel_cum;
      int chosen = -1, last_nonempty = -1;
      double cum_at_last = cum;
      for (int bin = 255; bin >= 0; --bin) {
        if (sh.hist_cnt[bin] == 0) continue;
        if (cum + sh.hist_mass[bin] > target) {
          chosen = bin;
          break;
        }
        last_nonempty = bin;
        cum_at_last = cum;
        cum += sh.hist_mass[bin];
      }
      if (chosen < 0) {  // rounding left the target at the very end: take the last element
        chosen = last_nonempty < 0 ? 0 : last_nonempty;
        cum = cum_at_last;
      }
      sh.sel_cum = cum;
      sh.sel_bin_cnt = sh.hist_cnt[chosen];
      sh.sel_bin_mass = sh.hist_mass[chosen];
      sh.sel_prefix = prefix | (static_cast<uint32_t>(chosen) << shift);
    }
    __syncthreads();
    prefix = sh.sel_prefix;
    mask |= 255u << shift;
  }
  const int cnt = sh.sel_bin_cnt;
  int j = 1;  // position within the tie group in walk (descending index) order
  if (cnt > 1) {
    const double w = sh.sel_bin_mass / cnt;
    const double jj = w > 0.0 ? floor((target - sh.sel_cum) / w) + 1.0 : 1.0;
    j = jj < 1.0 ? 1 : (jj > cnt ? cnt : static_cast<int>(jj));
  }
  *tau = prefix;
  *rank = cnt - j + 1;
}

// Index of the j-th (1-based, index order) element with pred(i); -1 if none.
template <typename FP>
__device__ int find_nth(int V, int j, FP pred, Shared& sh) {
  const int seg = (V + kThreads - 1) / kThreads;
  const int lo = threadIdx.x * seg, hi = min(V, lo + seg);
  int c = 0;
  for (int i = lo; i < hi; ++i) c += pred(i) ? 1 : 0;
  int total = 0;
  const int before = block_excl_scan_i(c, &total, sh);
  if (threadIdx.x == 0) sh.found_index = -1;
  __syncthreads();
  if (j <= total && before < j && before + c >= j) {
    int k = before;
    for (int i = lo; i < hi; ++i) {
      if (pred(i) && ++k == j) {
        sh.found_index = i;
        break;
      }
    }
  }
  __syncthreads();
  return sh.found_index;
}

// Logits rows up to this size (V ≤ 51,456 fp16 entries) are staged in LDS once, so the
// selection passes re-read LDS rather than HBM/L2.
constexpr int kRowCacheBytes = 100 * 1024 + 512;

template <typename T>
__global__ __launch_bounds__(kThreads) void sample_kernel(SampleArgs a) {
  __shared__ Shared sh;
  __shared__ __attribute__((aligned(16))) char s_row[kRowCacheBytes];
  __shared__ int s_cand[kCandMax];
  __shared__ __attribute__((aligned(16))) float s_candx[kCandMax];
  __shared__ uint32_t s_tkeys[kThreads];
  const int b = blockIdx.x;
  const int V = a.V;
  const bool gen = a.pos != nullptr;
  const int p_cur = gen ? a.pos[b] : (a.hist_len ? a.hist_len[b] - 1 : -1);
  Row<T> row;
  row.lg = static_cast<const T*>(a.logits) + b * a.logits_stride;
  row.V = V;
  row.pen = a.rep_penalty;
  row.temperature = a.temperature;
  row.use_pen = a.rep_penalty != 1.0f && a.tokens != nullptr;
  row.bitmap = sh.bitmap;

  if (row.use_pen) {
    for (int i = threadIdx.x; i < kBitmapWords; i += kThreads) sh.bitmap[i] = 0u;
    __syncthreads();
    const int64_t* hist = a.tokens + b * a.tok_stride;
    for (int i = threadIdx.x; i <= p_cur; i += kThreads) {
      const int64_t t = hist[i];
      if (t >= 0 && t < V) atomicOr(&sh.bitmap[t >> 5], 1u << (t & 31));
    }
    __syncthreads();
  }

  const bool sampled = a.temperature > 0.f;
  const bool use_p = a.top_p > 0.f && a.top_p < 1.f;
  const bool use_k = a.top_k > 0;
  const int k_eff = a.top_k < V ? a.top_k : V;
  double u = 0.0;
  if (sampled) {
    const long long ui = gen ? static_cast<long long>(p_cur + 1 - a.plen[b]) * a.B + b : b;
    u = a.uniforms[ui];
  }
  int chosen = -1;
  if constexpr (sizeof(T) == 2) {
    if (sampled && use_k && !use_p && sample_regs_applies(row, k_eff))
      chosen = sample_topk_regs(row, k_eff, u, sh, s_cand, s_candx);
  }
  if (chosen < 0) {
    // The selection passes re-read the row many times: with room for it, stage it in LDS
    // once (all 16-byte loads of the row in flight together) and let every pass read LDS.
    if (a.V * static_cast<int>(sizeof(T)) <= kRowCacheBytes) {
      T* cache = reinterpret_cast<T*>(s_row);
      constexpr int E = 16 / sizeof(T);
      const int nv = a.V / E;
      const bool aligned = (reinterpret_cast<uintptr_t>(row.lg) & 15) == 0;
      if (aligned) {
        typedef int iv4 __attribute__((ext_vector_type(4)));
        for (int i = threadIdx.x; i < nv; i += kThreads)
          reinterpret_cast<iv4*>(cache)[i] = reinterpret_cast<const iv4*>(row.lg)[i];
        for (int i = nv * E + threadIdx.x; i < a.V; i += kThreads) cache[i] = row.lg[i];
      } else {
        for (int i = threadIdx.x; i < a.V; i += kThreads) cache[i] = row.lg[i];
      }
      __syncthreads();
      row.lg = cache;
    }

    if (!sampled) {
      // argmax, first index among equal maxima
      float best = -INFINITY;
      int bi = 0x7fffffff;
      for (int i = threadIdx.x; i < V; i += kThreads) {
        const float x = row.base(i);
        if (x > best || (x == best && i < bi)) {
          best = x;
          bi = i;
        }
      }
  #pragma unroll
      for (int o = 32; o > 0; o >>= 1) {
        const float ob = __shfl_xor(best, o, 64);
        const int oi = __shfl_xor(bi, o, 64);
        if (ob > best || (ob == best && oi < bi)) {
          best = ob;
          bi = oi;
        }
      }
      __syncthreads();
      if ((threadIdx.x & 63) == 0) {
        sh.redf[threadIdx.x >> 6] = best;
        sh.redi[threadIdx.x >> 6] = bi;
      }
      __syncthreads();
      if (threadIdx.x == 0) {
        float bb = sh.redf[0];
        int ii = sh.redi[0];
        for (int w = 1; w < kWaves; ++w) {
          if (sh.redf[w] > bb || (sh.redf[w] == bb && sh.redi[w] < ii)) {
            bb = sh.redf[w];
            ii = sh.redi[w];
          }
        }
        sh.found_index = ii;
      }
      __syncthreads();
      chosen = sh.found_index;
    } else {
      if (use_k && !use_p) chosen = sample_topk_fast(row, k_eff, u, sh, s_cand, s_candx, s_tkeys);
      // top-k threshold on the temperature-scaled logits
      float thresh = -INFINITY;
      if (use_k && chosen < 0) {
        const uint32_t tk =
            select_kth_key(V, k_eff, [&](int i) { return fkey(row.scaled(i)); }, sh);
        const uint32_t bits = (tk & 0x80000000u) ? (tk & 0x7fffffffu) : ~tk;
        thresh = __uint_as_float(bits);
      }
      auto xm = [&](int i) {
        const float x = row.scaled(i);
        return (use_k && x < thresh) ? -1e9f : x;
      };
      if (use_k && !use_p && chosen < 0)
        chosen = sample_topk_candidates(row, thresh, u, sh, s_cand, s_candx);
      // max and Σ exp over the whole row, for the top-p and full-CDF draws
      float mx = -INFINITY, se = 0.f;
      if (chosen < 0) {
        for (int i = threadIdx.x; i < V; i += kThreads) mx = fmaxf(mx, xm(i));
        mx = block_max_f(mx, sh);
        for (int i = threadIdx.x; i < V; i += kThreads) se += expf(xm(i) - mx);
        se = block_sum_f(se, sh);
      }
      auto prob = [&](int i) { return expf(xm(i) - mx) / se; };
      auto keyp = [&](int i) { return fkey(prob(i)); };

      if (chosen >= 0) {
        // sampled among the top-k candidates
      } else if (use_p) {
        // Cut: first descending position whose running mass exceeds top_p.
        uint32_t tau1;
        int j1;
        select_by_mass(V, static_cast<double>(a.top_p), keyp, prob, [](int) { return true; }, &tau1,
                       &j1, sh);
        // Index of that element; kept = the elements before it in walk order:
        // key > τ1, or key == τ1 and index > cut index.
        const int cut = find_nth(V, j1, [&](int i) { return keyp(i) == tau1; }, sh);
        int ties1 = 0;
        for (int i = threadIdx.x; i < V; i += kThreads) ties1 += keyp(i) == tau1 ? 1 : 0;
        {
          int tot = 0;
          block_excl_scan_i(ties1, &tot, sh);
          ties1 = tot;
        }
        // Empty prefix (the crossing element is the top one) keeps that element alone.
        int above = 0;
        for (int i = threadIdx.x; i < V; i += kThreads) above += keyp(i) > tau1 ? 1 : 0;
        {
          int tot = 0;
          block_excl_scan_i(above, &tot, sh);
          above = tot;
        }
        const bool single = (above == 0 && j1 == ties1);  // cut is the largest tied index
        auto kept = [&](int i) {
          const uint32_t k = keyp(i);
          if (single) return i == cut;
          return k > tau1 || (k == tau1 && i > cut);
        };
        float ks = 0.f;
        for (int i = threadIdx.x; i < V; i += kThreads) ks += kept(i) ? prob(i) : 0.f;
        ks = block_sum_f(ks, sh);
        auto q = [&](int i) { return prob(i) / ks; };
        double tq = 0.0;
        for (int i = threadIdx.x; i < V; i += kThreads)
          tq += kept(i) ? static_cast<double>(q(i)) : 0.0;
        double total = 0.0;
        block_excl_scan_d(tq, &total, sh);
        uint32_t tau2;
        int j2;
        // The renormalised list keeps the order of p (generate.py:50-58).
        select_by_mass(V, u * total, keyp, q, kept, &tau2, &j2, sh);
        chosen = find_nth(V, j2, [&](int i) { return kept(i) && keyp(i) == tau2; }, sh);
      } else {
        // Index-order float64 CDF; first i with cdf[i] / cdf[-1] > u.
        const int seg = (V + kThreads - 1) / kThreads;
        const int lo = threadIdx.x * seg, hi = min(V, lo + seg);
        double part = 0.0;
        for (int i = lo; i < hi; ++i) part += static_cast<double>(prob(i));
        double total = 0.0;
        double run = block_excl_scan_d(part, &total, sh);
        if (threadIdx.x == 0) sh.found_index = 0x7fffffff;
        __syncthreads();
        for (int i = lo; i < hi; ++i) {
          run += static_cast<double>(prob(i));
          if (run / total > u) {
            atomicMin(&sh.found_index, i);
            break;
          }
        }
        __syncthreads();
        if (sh.found_index == 0x7fffffff) {
          // none hit (the running sums end an ulp below `total`): the reference's
          // searchsorted over cdf / cdf[-1] lands on the last index of nonzero mass
          __syncthreads();
          if (threadIdx.x == 0) sh.found_index = -1;
          __syncthreads();
          for (int i = hi - 1; i >= lo; --i)
            if (prob(i) > 0.f) {
              atomicMax(&sh.found_index, i);
              break;
            }
          __syncthreads();
        }
        chosen = sh.found_index < 0 ? V - 1 : sh.found_index;
      }
    }
  }  // general path

  if (threadIdx.x == 0) {
    if (gen) {
      a.tokens[b * a.tok_stride + p_cur + 1] = chosen;
      a.pos[b] = p_cur + 1;
    }
    if (a.out_ids) a.out_ids[b] = chosen;
  }
}

}  // namespace

int launch_sample(int dt, const SampleArgs& a, hipStream_t st) {
  if (a.B == 0) return 0;
  NML_REQUIRE(a.temperature <= 0.f || a.uniforms != nullptr, "sample: uniforms required when T > 0");
  NML_REQUIRE(a.pos == nullptr || (a.tokens != nullptr && a.plen != nullptr),
              "sample: generation mode needs the token history and prompt lengths");
  NML_REQUIRE(a.rep_penalty == 1.0f || a.V <= kBitmapWords * 32,
              "sample: repetition penalty supports vocab ≤ %d", kBitmapWords * 32);
  if (dt == F16)
    sample_kernel<half_t><<<a.B, kThreads, 0, st>>>(a);
  else
    sample_kernel<float><<<a.B, kThreads, 0, st>>>(a);
  NML_LAUNCHED();
  return 0;
}

}  // namespace nml
