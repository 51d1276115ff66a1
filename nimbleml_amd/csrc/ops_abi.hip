// Single-op entry points of the C-ABI (the `*_device` family). Each validates its
// shapes on the host, then launches on the library stream.
#include <cmath>
#include <mutex>
#include <vector>

#include "kernels.hpp"
#include "nimbleml_hip.h"

using namespace nml;

// Fixed device scratch of nml_tied_ce_forward_device_noalloc: 32 MiB, held by every GPU the
// library runs on until the process ends. All calls on one GPU share it (and it keeps the
// last call's contents), so such calls must not overlap on one GPU: issue them on one
// stream, or synchronise between them.
constexpr size_t kNoAllocScratchBytes = size_t(32) << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace {

// Grow-only scratch for the ops that need temporaries.
struct Scratch {
  void* p = nullptr;
  size_t bytes = 0;
  int ensure(size_t want) {
    if (want <= bytes) return 0;
    if (p) {
      NML_HIP(hipStreamSynchronize(nml::stream()));
      NML_HIP(hipFree(p));
      p = nullptr;
      bytes = 0;
    }
    NML_HIP(hipMalloc(&p, want));
    bytes = want;
    return 0;
  }
};
Scratch g_scratch;

int check_dtype(int dt) {
  NML_REQUIRE(dt == F32 || dt == F16, "dtype must be 0 (float32) or 1 (float16), got %d", dt);
  return 0;
}

// lse = m + log(max(l, 1e-20)): the softmax statistics of the reference's flash kernel
// (sdpa_cuda.cu:84-86) as the log-sum-exp the attention backward kernels take.
__global__ void lse_from_ml_kernel(const float* __restrict__ m, const float* __restrict__ l,
                                   float* __restrict__ lse, long long n) {
  const long long i = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) lse[i] = m[i] + logf(fmaxf(l[i], 1e-20f));
}

// Rows of [dq | dk | dv] (rows, 3·dk) → three (rows, dk) arrays.
__global__ void split3_kernel(const float* __restrict__ src, float* __restrict__ a,
                              float* __restrict__ b, float* __restrict__ c, long long rows,
                              int dk) {
  const long long i = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= rows * dk) return;
  const long long r = i / dk, j = i % dk;
  const float* s = src + r * 3 * dk;
  a[i] = s[j];
  b[i] = s[dk + j];
  c[i] = s[2 * dk + j];
}

int attn_shape_ok(size_t bh, size_t seq, size_t dk) {
  NML_REQUIRE(dk >= 1 && dk <= (size_t)kMaxHeadDim, "attention: head_dim %zu outside [1, %d]", dk,
              kMaxHeadDim);
  NML_REQUIRE(bh <= 65535 && bh * seq <= 0x7fffffff, "attention: %zu × %zu rows too many", bh,
              seq);
  return 0;
}

// Scratch of one tied cross-entropy pass over row chunks of `chunk` rows: the chunk's
// logits, its per-row losses and validity flags, then the error word and the float64
// accumulators.
size_t ce_scratch_bytes(size_t chunk, size_t vocab, size_t es) {
  const size_t lb = ((chunk * vocab * es + 255) / 256) * 256;
  const size_t rb = ((chunk * 4 + 255) / 256) * 256;
  return lb + 2 * rb + 256;
}

__global__ void zero_words_kernel(unsigned* p, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0u;
}

// Mean tied cross-entropy in row chunks of at most `chunk` rows with the scratch at ws
// (ce_scratch_bytes(chunk, vocab, es) bytes). Allocates nothing; returns after the device
// finishes, the mean in *loss.
int tied_ce(const void* hidden, const void* weights, const int64_t* labels, size_t rows,
            size_t dim, size_t vocab, int64_t ignore_index, int has_ignore, double* loss, int dtype,
            void* ws, size_t chunk) {
  NML_REQUIRE(rows <= 0x7fffffff && vocab <= 0x7fffffff && dim <= 0x7fffffff,
              "cross-entropy: sizes out of range");
  const size_t es = dtype_size(dtype);
  const size_t lbytes = ((chunk * vocab * es + 255) / 256) * 256;
  const size_t rbytes = ((chunk * 4 + 255) / 256) * 256;
  char* base = static_cast<char*>(ws);
  void* logits = base;
  float* row_loss = reinterpret_cast<float*>(base + lbytes);
  int* row_valid = reinterpret_cast<int*>(base + lbytes + rbytes);
  int* err = reinterpret_cast<int*>(base + lbytes + 2 * rbytes);
  double* acc = reinterpret_cast<double*>(base + lbytes + 2 * rbytes + 64);
  hipStream_t st = nml::stream();
  // err and the two accumulators start at zero (a fill kernel, no memset node)
  zero_words_kernel<<<1, 64, 0, st>>>(reinterpret_cast<unsigned*>(base + lbytes + 2 * rbytes), 32);
  NML_LAUNCHED();
  for (size_t r0 = 0; r0 < rows; r0 += chunk) {
    const size_t n = (rows - r0 < chunk) ? rows - r0 : chunk;
    LinearArgs a{};
    a.x = static_cast<const char*>(hidden) + r0 * dim * es;
    a.lda = (long long)dim;
    a.w = weights;
    a.out = logits;
    a.M = (int)n;
    a.N = (int)vocab;
    a.K = (int)dim;
    a.epi = EPI_NONE;
    NML_TRY(launch_linear(dtype, a, st));
    NML_TRY(launch_ce_rows(dtype, logits, (int)n, (int)vocab, labels + r0, ignore_index,
                           has_ignore, row_loss, row_valid, err, st));
    NML_TRY(launch_ce_reduce(row_loss, row_valid, (int)n, acc, r0 > 0 ? 1 : 0, st));
  }
  NML_TRY(launch_ce_finalize(acc, acc + 2, st));
  double host[3];
  int herr = 0;
  NML_HIP(hipMemcpyAsync(host, acc, sizeof(host), hipMemcpyDeviceToHost, st));
  NML_HIP(hipMemcpyAsync(&herr, err, sizeof(int), hipMemcpyDeviceToHost, st));
  NML_HIP(hipStreamSynchronize(st));
  NML_REQUIRE(herr == 0, "cross-entropy: label out of range [0, %zu)", vocab);
  *loss = host[2];
  return 0;
}

// Library-owned workspace of nml_decode_attention_device: the rows' last positions
// (int32), then the decode kernels' partials. The grouped kernel leaves its partial slots
// zeroed after every launch, so the buffer is cleared once, when it is (re)allocated.
struct DecodeWs {
  void* p = nullptr;
  size_t bytes = 0;
  int ensure(size_t want, hipStream_t st) {
    if (want <= bytes) return 0;
    if (p) {
      NML_HIP(hipStreamSynchronize(st));
      NML_HIP(hipFree(p));
      p = nullptr;
      bytes = 0;
    }
    NML_HIP(hipMalloc(&p, want));
    bytes = want;
    NML_HIP(hipMemsetAsync(p, 0, want, st));
    return 0;
  }
};
DecodeWs g_decode_ws;

// pos[b] = lens[b] − 1 for the decode kernels, with lens clamped into [1, max_seq] so no
// key past the cache is read; a clamped length sets bit 0 of *err.
__global__ void lens_to_pos_kernel(const int32_t* __restrict__ lens, int32_t* __restrict__ pos,
                                   int n, int max_seq, int* __restrict__ err) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int len = lens[i];
  const int c = len < 1 ? 1 : (len > max_seq ? max_seq : len);
  if (c != len && err) __hip_atomic_fetch_or(err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  pos[i] = c - 1;
}

constexpr int kMaxDevices = 64;
std::mutex g_noalloc_mu;
void* g_noalloc_ptr[kMaxDevices] = {};

// The device address of `scratch` on the current device, looked up once per device (the
// host-side name `scratch` is not a device address and must never reach a kernel).
int noalloc_scratch(void** out) {
  int dev = 0;
  NML_HIP(hipGetDevice(&dev));
  NML_REQUIRE(dev >= 0 && dev < kMaxDevices, "no-alloc scratch: device %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_noalloc_mu);
  if (!g_noalloc_ptr[dev]) {
    void* p = nullptr;
    NML_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    NML_REQUIRE(p != nullptr, "no-alloc scratch: no device address on device %d", dev);
    g_noalloc_ptr[dev] = p;
  }
  *out = g_noalloc_ptr[dev];
  return 0;
}

}  // namespace

extern "C" {

int nml_rmsnorm_forward_device(const void* x, const void* gamma, void* out, float* ms, float* rms,
                               size_t rows, size_t dim, float eps, int dtype) {
  NML_TRY(check_dtype(dtype));
  NML_REQUIRE(dim > 0 && dim <= (1u << 20), "rmsnorm: dim %zu out of range", dim);
  NML_REQUIRE(rows <= 0x7fffffff, "rmsnorm: too many rows");
  return launch_rmsnorm(dtype, x, gamma, out, ms, rms, (int)rows, (int)dim, eps, nml::stream());
}

int nml_gelu_forward_device(const void* x, void* out, float* tanh_u, size_t n, int dtype) {
  NML_TRY(check_dtype(dtype));
  return launch_gelu(dtype, x, out, tanh_u, n, nml::stream());
}

int nml_embedding_gather_device(const void* weights, const void* pos_weights, const int64_t* ids,
                                void* out, size_t batch, size_t seq, size_t dim, size_t vocab,
                                size_t max_pos, const int32_t* pos_offsets, int* err, int dtype) {
  NML_TRY(check_dtype(dtype));
  NML_REQUIRE(pos_weights != nullptr, "embedding: position table required");
  NML_REQUIRE(batch * seq <= 0x7fffffff, "embedding: too many rows");
  return launch_embed(dtype, ids, weights, pos_weights, pos_offsets, out, (int)batch, (int)seq,
                      (int)dim, (int)vocab, (int)max_pos, err, nml::stream());
}

int nml_linear_device(const void* x, size_t ld_x, const void* w_t, const void* bias,
                      const void* resid, void* out, size_t rows, size_t in_f, size_t out_f,
                      int epilogue, int dtype) {
  NML_TRY(check_dtype(dtype));
  NML_REQUIRE(epilogue >= EPI_NONE && epilogue <= EPI_BIAS_RESID,
              "linear: epilogue %d not available here", epilogue);
  NML_REQUIRE(ld_x >= in_f, "linear: ld_x < in_f");
  NML_TRY(linear_reserve_workspace(4096));
  LinearArgs a{};
  a.x = x;
  a.lda = (long long)ld_x;
  a.w = w_t;
  a.bias = bias;
  a.resid = resid;
  a.out = out;
  a.M = (int)rows;
  a.N = (int)out_f;
  a.K = (int)in_f;
  a.epi = epilogue;
  return launch_linear(dtype, a, nml::stream());
}

int nml_causal_attention_device(const void* q, const void* k, const void* v, void* out, size_t bh,
                                size_t seq, size_t dk, float scale_div, int dtype) {
  NML_TRY(check_dtype(dtype));
  NML_TRY(attn_shape_ok(bh, seq, dk));
  AttnArgs a{};
  a.q = q;
  a.k = k;
  a.v = v;
  a.out = out;
  a.kv_stride_b = (long long)(seq * dk);
  a.B = (int)bh;
  a.H = 1;
  a.S = (int)seq;
  a.dk = (int)dk;
  a.scale = scale_div;
  return launch_attention_prefill(dtype, a, nml::stream());
}

int nml_sdpa_forward_device(const void* q, const void* k, const void* v, const void* mask,
                            void* out, size_t bh, size_t seq, size_t dk, float scale_div,
                            int causal, int dtype) {
  NML_TRY(check_dtype(dtype));
  NML_TRY(attn_shape_ok(bh, seq, dk));
  NML_REQUIRE(!causal || mask == nullptr, "sdpa_forward: a causal call takes no mask");
  AttnArgs a{};
  a.q = q;
  a.k = k;
  a.v = v;
  a.out = out;
  a.kv_stride_b = (long long)(seq * dk);
  a.B = (int)bh;
  a.H = 1;
  a.S = (int)seq;
  a.dk = (int)dk;
  a.scale = scale_div;
  a.full = causal ? 0 : 1;
  a.mask = mask;
  return launch_attention_prefill(dtype, a, nml::stream());
}

int nml_flash_sdpa_forward_device(const float* q, const float* k, const float* v, float* out,
                                  float* m, float* l, size_t bh, size_t seq, size_t dk,
                                  float scale) {
  NML_TRY(attn_shape_ok(bh, seq, dk));
  NML_REQUIRE(scale > 0.f && std::isfinite(scale), "flash_sdpa_forward: scale must be positive");
  NML_REQUIRE(m != nullptr && l != nullptr, "flash_sdpa_forward: m and l are required");
  AttnArgs a{};
  a.q = q;
  a.k = k;
  a.v = v;
  a.out = out;
  a.kv_stride_b = (long long)(seq * dk);
  a.B = (int)bh;
  a.H = 1;
  a.S = (int)seq;
  a.dk = (int)dk;
  a.scale = 1.0f / scale;  // the kernels divide the scores; the reference multiplies
  a.m_out = m;
  a.l_out = l;
  return launch_attention_prefill(F32, a, nml::stream());
}

int nml_decode_attention_device(const void* q, const void* kcache, const void* vcache,
                                const int32_t* lens, void* out, size_t batch, size_t heads,
                                size_t max_seq, size_t dk, float scale_div, int* err, int dtype) {
  NML_TRY(check_dtype(dtype));
  NML_REQUIRE(dk >= 1 && dk <= (size_t)kMaxHeadDim, "decode attention: head_dim %zu outside [1, %d]",
              dk, kMaxHeadDim);
  NML_REQUIRE(batch * heads <= 65535, "decode attention: %zu × %zu (row, head) pairs too many", batch,
              heads);
  NML_REQUIRE(max_seq >= 1 && max_seq <= 65536, "decode attention: max_seq %zu outside [1, 65536]",
              max_seq);
  NML_REQUIRE(scale_div > 0.f && std::isfinite(scale_div),
              "decode attention: scale_div must be positive");
  NML_REQUIRE(lens != nullptr, "decode attention: lens is required");
  if (batch == 0 || heads == 0) return 0;
  hipStream_t st = nml::stream();
  const size_t pos_b = ((batch * 4 + 255) / 256) * 256;
  NML_TRY(g_decode_ws.ensure(
      pos_b + attention_decode_workspace((int)batch, (int)heads, (int)dk, (int)max_seq), st));
  int32_t* pos = static_cast<int32_t*>(g_decode_ws.p);
  lens_to_pos_kernel<<<(unsigned)((batch + 255) / 256), 256, 0, st>>>(lens, pos, (int)batch,
                                                                     (int)max_seq, err);
  NML_LAUNCHED();
  AttnArgs a{};
  a.q = q;
  a.k = kcache;
  a.v = vcache;
  a.out = out;
  a.kv_stride_b = (long long)(heads * max_seq * dk);
  a.kv_stride_h = (long long)(max_seq * dk);
  a.B = (int)batch;
  a.H = (int)heads;
  a.S = 1;
  a.dk = (int)dk;
  a.scale = scale_div;
  return launch_attention_decode(dtype, a, pos, (int)max_seq, static_cast<char*>(g_decode_ws.p) + pos_b,
                                 st);
}

int nml_flash_sdpa_backward_device(const float* grad_out, const float* q, const float* k,
                                   const float* v, const float* m, const float* l, float* grad_q,
                                   float* grad_k, float* grad_v, size_t bh, size_t seq, size_t dk,
                                   float scale) {
  NML_TRY(attn_shape_ok(bh, seq, dk));
  NML_REQUIRE(scale > 0.f && std::isfinite(scale), "flash_sdpa_backward: scale must be positive");
  const size_t rows = bh * seq;
  if (rows == 0) return 0;
  // scratch: the forward output (rows·dk), lse and the per-row dot (rows each), and the
  // three gradients side by side (rows·3dk)
  const size_t o_b = ((rows * dk * 4 + 255) / 256) * 256, r_b = ((rows * 4 + 255) / 256) * 256;
  NML_TRY(g_scratch.ensure(o_b + 2 * r_b + 3 * o_b));
  char* base = static_cast<char*>(g_scratch.p);
  float* o = reinterpret_cast<float*>(base);
  float* lse = reinterpret_cast<float*>(base + o_b);
  float* dvec = reinterpret_cast<float*>(base + o_b + r_b);
  float* dqkv = reinterpret_cast<float*>(base + o_b + 2 * r_b);
  hipStream_t st = nml::stream();
  AttnArgs fa{};
  fa.q = q;
  fa.k = k;
  fa.v = v;
  fa.out = o;
  fa.kv_stride_b = (long long)(seq * dk);
  fa.B = (int)bh;
  fa.H = 1;
  fa.S = (int)seq;
  fa.dk = (int)dk;
  fa.scale = 1.0f / scale;
  NML_TRY(launch_attention_prefill(F32, fa, st));
  lse_from_ml_kernel<<<(unsigned)((rows + 255) / 256), 256, 0, st>>>(m, l, lse, (long long)rows);
  NML_LAUNCHED();
  AttnBwdArgs ba{};
  ba.q = q;
  ba.k = k;
  ba.v = v;
  ba.o = o;
  ba.dout = grad_out;
  ba.lse = lse;
  ba.dvec = dvec;
  ba.dqkv = dqkv;
  ba.B = (int)bh;
  ba.H = 1;
  ba.S = (int)seq;
  ba.dk = (int)dk;
  ba.scale = 1.0f / scale;
  NML_TRY(launch_attention_backward(F32, ba, st));
  split3_kernel<<<(unsigned)((rows * dk + 255) / 256), 256, 0, st>>>(dqkv, grad_q, grad_k, grad_v,
                                                                   (long long)rows, (int)dk);
  NML_LAUNCHED();
  return 0;
}

int nml_rmsnorm_backward_device(const float* grad, const float* x, const float* gamma,
                                const float* ms, const float* rms, float* grad_x,
                                float* grad_gamma, size_t rows, size_t dim, float eps) {
  (void)ms;
  (void)rms;  // recomputed from x with the forward's own arithmetic
  NML_REQUIRE(dim > 0 && dim <= 8192, "rmsnorm backward: dim %zu outside (0, 8192]", dim);
  NML_REQUIRE(rows <= 0x7fffffff, "rmsnorm backward: too many rows");
  hipStream_t st = nml::stream();
  NML_HIP(hipMemsetAsync(grad_gamma, 0, dim * sizeof(float), st));
  if (rows == 0) return 0;
  const size_t parts = (size_t)rmsnorm_bwd_parts((int)rows) + 1;
  NML_TRY(g_scratch.ensure(parts * dim * sizeof(float)));
  return launch_rmsnorm_bwd(F32, grad, x, gamma, grad_x, 0, grad_gamma,
                            static_cast<float*>(g_scratch.p), (int)rows, (int)dim, eps, st);
}

int nml_linear_backward_device(const void* dy, const void* x, const void* w_t, void* dx,
                               float* dw_t, float* db, size_t rows, size_t in_features,
                               size_t out_features, const void* gelu_pre, int dtype) {
  NML_TRY(check_dtype(dtype));
  NML_REQUIRE(rows <= 0x7fffffff && in_features <= 0x7fffffff && out_features <= 0x7fffffff,
              "linear backward: shape too large");
  NML_REQUIRE(!gelu_pre || dx, "linear backward: gelu_pre given without dx");
  if (rows == 0 || in_features == 0 || out_features == 0) return 0;
  const int M = (int)rows, K = (int)in_features, N = (int)out_features;
  hipStream_t st = nml::stream();
  auto gbw = [](const void* a, long long lda, const void* b, long long ldb, void* c,
                long long ldc, int m, int n, int k, const void* aux, long long ldaux) {
    GemmBwdArgs g{};
    g.a = a;
    g.lda = lda;
    g.b = b;
    g.ldb = ldb;
    g.c = c;
    g.ldc = ldc;
    g.aux = aux;
    g.ldaux = ldaux;
    g.M = m;
    g.N = n;
    g.K = k;
    return g;
  };
  if (dx)  // dx(r, i) = Σ_o dy(r, o)·W(o, i) [· gelu'(pre(r, i))]
    NML_TRY(launch_gemm_bwd(dtype, gbw(dy, N, w_t, K, dx, K, M, K, N, gelu_pre, K), true, false,
                            gelu_pre ? GB_GELU : GB_SET, st));
  if (dw_t)  // dW(o, i) += Σ_r dy(r, o)·x(r, i)
    NML_TRY(launch_gemm_bwd(dtype, gbw(dy, N, x, K, dw_t, K, N, K, M, nullptr, 0), false, false,
                            GB_ADD, st));
  if (db) {  // db(o) += Σ_r dy(r, o)
    NML_TRY(g_scratch.ensure((size_t)colsum_parts(M) * N * sizeof(float)));
    NML_TRY(launch_colsum(dtype, dy, N, M, N, db, static_cast<float*>(g_scratch.p), st));
  }
  NML_HIP(hipStreamSynchronize(st));
  return 0;
}

int nml_rmsnorm_backward_typed_device(const void* grad, const void* x, const void* gamma,
                                      void* grad_x, float* grad_gamma, size_t rows, size_t dim,
                                      float eps, int dtype) {
  NML_TRY(check_dtype(dtype));
  NML_REQUIRE(dim > 0 && dim <= 8192, "rmsnorm backward: dim %zu outside (0, 8192]", dim);
  NML_REQUIRE(rows <= 0x7fffffff, "rmsnorm backward: too many rows");
  if (rows == 0) return 0;
  hipStream_t st = nml::stream();
  const size_t parts = (size_t)rmsnorm_bwd_parts((int)rows) + 1;
  NML_TRY(g_scratch.ensure(parts * dim * sizeof(float)));
  NML_TRY(launch_rmsnorm_bwd(dtype, grad, x, gamma, grad_x, 0, grad_gamma,
                             static_cast<float*>(g_scratch.p), (int)rows, (int)dim, eps, st));
  NML_HIP(hipStreamSynchronize(st));
  return 0;
}

int nml_embedding_backward_device(const void* grad, const int64_t* ids, float* grad_weights,
                                  size_t rows, size_t dim, size_t vocab, int dtype) {
  NML_TRY(check_dtype(dtype));
  NML_REQUIRE(rows <= 0x7fffffff && dim <= 0x7fffffff && vocab <= 0x7fffffff,
              "embedding backward: shape too large");
  if (rows == 0 || dim == 0) return 0;
  hipStream_t st = nml::stream();
  NML_TRY(launch_embed_backward(dtype, grad, ids, grad_weights, nullptr, 1, (int)rows, (int)dim,
                                (int)vocab, st));
  NML_HIP(hipStreamSynchronize(st));
  return 0;
}

int nml_tied_ce_forward_device(const void* hidden, const void* weights, const int64_t* labels,
                               size_t rows, size_t dim, size_t vocab, int64_t ignore_index,
                               int has_ignore, double* loss, int dtype) {
  NML_TRY(check_dtype(dtype));
  const size_t es = dtype_size(dtype);
  size_t chunk = rows ? rows : 1;
  const size_t cap = (size_t)256 << 20;
  while (chunk > 1 && chunk * vocab * es > cap) chunk = (chunk + 1) / 2;
  NML_TRY(g_scratch.ensure(ce_scratch_bytes(chunk, vocab, es)));
  return tied_ce(hidden, weights, labels, rows, dim, vocab, ignore_index, has_ignore, loss, dtype,
                 g_scratch.p, chunk);
}

int nml_tied_ce_forward_device_noalloc(const void* hidden, const void* weights,
                                       const int64_t* labels, size_t rows, size_t dim,
                                       size_t vocab, int64_t ignore_index, int has_ignore,
                                       double* loss, int dtype) {
  NML_TRY(check_dtype(dtype));
  const size_t es = dtype_size(dtype);
  NML_REQUIRE(ce_scratch_bytes(1, vocab, es) <= kNoAllocScratchBytes,
              "tied cross-entropy (no-alloc): one row of %zu logits needs %zu bytes of scratch, "
              "more than the fixed %zu",
              vocab, ce_scratch_bytes(1, vocab, es), kNoAllocScratchBytes);
  size_t chunk = rows ? rows : 1;
  while (chunk > 1 && ce_scratch_bytes(chunk, vocab, es) > kNoAllocScratchBytes)
    chunk = (chunk + 1) / 2;
  void* ws = nullptr;
  NML_TRY(noalloc_scratch(&ws));
  return tied_ce(hidden, weights, labels, rows, dim, vocab, ignore_index, has_ignore, loss, dtype,
                 ws, chunk);
}

int nml_sample_device(const void* logits, size_t batch, size_t vocab, float temperature, int top_k,
                      float top_p, float repetition_penalty, const double* u,
                      const int64_t* history, size_t history_stride, const int32_t* hist_len,
                      int64_t* out_ids, int dtype) {
  NML_TRY(check_dtype(dtype));
  SampleArgs a{};
  a.logits = logits;
  a.logits_stride = (long long)vocab;
  a.B = (int)batch;
  a.V = (int)vocab;
  a.temperature = temperature;
  a.top_k = top_k;
  a.top_p = top_p;
  a.rep_penalty = repetition_penalty;
  a.uniforms = u;
  a.tokens = const_cast<int64_t*>(history);
  a.tok_stride = (long long)history_stride;
  a.pos = nullptr;
  a.plen = nullptr;
  a.hist_len = history ? hist_len : nullptr;
  a.out_ids = out_ids;
  return launch_sample(dtype, a, nml::stream());
}

}  // extern "C"
