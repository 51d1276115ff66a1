// Cross-entropy over tied-LM-head logits (kernels/fused_crossentropy.py:14-30):
//   loss = mean_r( max_r + log Σ_v exp(l[r,v] − max_r) − l[r, y_r] )
// fp16: l − max and exp are fp16 ops (one rounding each), the sum accumulates in
// fp32 (`dtype=acc`, :17-21). Rows whose label equals ignore_index are dropped
// (losses/_ce_prepare.py:46-69); no valid row gives 0 (…:60-68).
#include "kernels.hpp"

namespace nml {

namespace {

template <typename T>
__global__ __launch_bounds__(256) void ce_rows_kernel(const T* __restrict__ logits, int V,
                                                      const int64_t* __restrict__ labels,
                                                      long long ignore_index, int has_ignore,
                                                      float* __restrict__ row_loss,
                                                      int* __restrict__ row_valid,
                                                      int* __restrict__ err) {
#pragma clang fp contract(off)
  __shared__ float red[16];
  const int r = blockIdx.x;
  const T* l = logits + static_cast<size_t>(r) * V;
  const int64_t y = labels[r];
  if (has_ignore && y == ignore_index) {
    if (threadIdx.x == 0) {
      row_loss[r] = 0.f;
      row_valid[r] = 0;
    }
    return;
  }
  if (y < 0 || y >= V) {
    if (threadIdx.x == 0) {
      atomicOr(err, 2);
      row_loss[r] = 0.f;
      row_valid[r] = 0;
    }
    return;
  }
  float mx = -INFINITY;
  for (int v = threadIdx.x; v < V; v += blockDim.x) mx = fmaxf(mx, static_cast<float>(l[v]));
  mx = wave_max(mx);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  if (lane == 0) red[w] = mx;
  __syncthreads();
  mx = red[0];
  for (int i = 1; i < (int)(blockDim.x >> 6); ++i) mx = fmaxf(mx, red[i]);
  float s = 0.f;
  for (int v = threadIdx.x; v < V; v += blockDim.x)
    s += rnd<T>(expf(rnd<T>(static_cast<float>(l[v]) - mx)));
  s = block_sum(s, red);
  if (threadIdx.x == 0) {
    const float lse = mx + logf(s);
    row_loss[r] = lse - static_cast<float>(l[y]);
    row_valid[r] = 1;
  }
}

// Rows of the fused head (EPI_CE partials), one wave per row: M = max of the tile maxima,
// S = Σ_t s_t·exp(mx_t − M) (tiles in lane-strided order, then the wave sum), and the
// row's loss lse − logit[label] with lse = M + log S, as ce_rows_kernel forms it.
__global__ __launch_bounds__(256) void ce_combine_kernel(const float2* __restrict__ part, int tiles_n,
                                                         const float* __restrict__ label_logit,
                                                         int rows, int V,
                                                         const int64_t* __restrict__ labels,
                                                         long long ignore_index, int has_ignore,
                                                         float* __restrict__ row_loss,
                                                         int* __restrict__ row_valid,
                                                         int* __restrict__ err) {
#pragma clang fp contract(off)
  const int r = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (r >= rows) return;
  const int64_t y = labels[r];
  const bool ignored = has_ignore && y == ignore_index;
  if (ignored || y < 0 || y >= V) {
    if (lane == 0) {
      if (!ignored) atomicOr(err, 2);
      row_loss[r] = 0.f;
      row_valid[r] = 0;
    }
    return;
  }
  const float2* p = part + static_cast<size_t>(r) * tiles_n;
  float mx = -INFINITY;
  for (int t = lane; t < tiles_n; t += 64) mx = fmaxf(mx, p[t].x);
  mx = wave_max(mx);
  float s = 0.f;
  for (int t = lane; t < tiles_n; t += 64) {
    const float2 v = p[t];
    s += v.y * expf(v.x - mx);
  }
  s = wave_sum(s);
  if (lane == 0) {
    const float lse = mx + logf(s);
    row_loss[r] = lse - label_logit[r];
    row_valid[r] = 1;
  }
}

// Single block: accumulate Σ valid row losses and the count into sum_count[0..1].
__global__ __launch_bounds__(1024) void ce_reduce_kernel(const float* __restrict__ row_loss,
                                                         const int* __restrict__ row_valid,
                                                         int rows, double* __restrict__ sum_count,
                                                         int accumulate) {
  __shared__ double rs[16], rc[16];
  double s = 0.0, c = 0.0;
  for (int i = threadIdx.x; i < rows; i += blockDim.x) {
    if (row_valid[i]) {
      s += static_cast<double>(row_loss[i]);
      c += 1.0;
    }
  }
  s = wave_sum_d(s);
  c = wave_sum_d(c);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  if (lane == 0) {
    rs[w] = s;
    rc[w] = c;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    double ts = 0.0, tc = 0.0;
    for (int i = 0; i < (int)(blockDim.x >> 6); ++i) {
      ts += rs[i];
      tc += rc[i];
    }
    if (accumulate) {
      sum_count[0] += ts;
      sum_count[1] += tc;
    } else {
      sum_count[0] = ts;
      sum_count[1] = tc;
    }
  }
}

__global__ void ce_finalize_kernel(const double* __restrict__ sum_count, double* __restrict__ loss) {
  if (threadIdx.x == 0) loss[0] = sum_count[1] > 0.0 ? sum_count[0] / sum_count[1] : 0.0;
}

}  // namespace

int launch_ce_rows(int dt, const void* logits, int rows, int V, const int64_t* labels,
                   long long ignore_index, int has_ignore, float* row_loss, int* row_valid,
                   int* err, hipStream_t st) {
  if (rows == 0) return 0;
  if (dt == F16)
    ce_rows_kernel<half_t><<<rows, 256, 0, st>>>((const half_t*)logits, V, labels, ignore_index,
                                                 has_ignore, row_loss, row_valid, err);
  else
    ce_rows_kernel<float><<<rows, 256, 0, st>>>((const float*)logits, V, labels, ignore_index,
                                                has_ignore, row_loss, row_valid, err);
  NML_LAUNCHED();
  return 0;
}

int launch_ce_combine(const float2* part, int tiles_n, const float* label_logit, int rows, int V,
                      const int64_t* labels, long long ignore_index, int has_ignore,
                      float* row_loss, int* row_valid, int* err, hipStream_t st) {
  if (rows == 0) return 0;
  ce_combine_kernel<<<(rows + 3) / 4, 256, 0, st>>>(part, tiles_n, label_logit, rows, V, labels,
                                                    ignore_index, has_ignore, row_loss, row_valid,
                                                    err);
  NML_LAUNCHED();
  return 0;
}

int launch_ce_reduce(const float* row_loss, const int* row_valid, int rows, double* sum_count,
                     int accumulate, hipStream_t st) {
  ce_reduce_kernel<<<1, 1024, 0, st>>>(row_loss, row_valid, rows, sum_count, accumulate);
  NML_LAUNCHED();
  return 0;
}

int launch_ce_finalize(const double* sum_count, double* loss, hipStream_t st) {
  ce_finalize_kernel<<<1, 64, 0, st>>>(sum_count, loss);
  NML_LAUNCHED();
  return 0;
}

}  // namespace nml
