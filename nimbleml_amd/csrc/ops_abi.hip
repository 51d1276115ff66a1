// Single-op entry points of the C-ABI (the `*_device` family). Each validates its
// shapes on the host, then launches on the library stream.
#include <vector>

#include "kernels.hpp"
#include "nimbleml_hip.h"

using namespace nml;

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

int nml_flash_sdpa_forward_device(const void* q, const void* k, const void* v, void* out,
                                  size_t bh, size_t seq, size_t dk, float scale, int dtype) {
  NML_TRY(check_dtype(dtype));
  AttnArgs a{};
  a.q = q;
  a.k = k;
  a.v = v;
  a.out = out;
  a.pos_base = nullptr;
  a.kv_stride_b = (long long)(seq * dk);
  a.kv_stride_h = 0;
  a.B = (int)bh;
  a.H = 1;
  a.S = (int)seq;
  a.dk = (int)dk;
  a.scale = scale;
  return launch_attention_prefill(dtype, a, nml::stream());
}

int nml_tied_ce_forward_device(const void* hidden, const void* weights, const int64_t* labels,
                               size_t rows, size_t dim, size_t vocab, int64_t ignore_index,
                               int has_ignore, double* loss, int dtype) {
  NML_TRY(check_dtype(dtype));
  const size_t es = dtype_size(dtype);
  size_t chunk = rows ? rows : 1;
  const size_t cap = (size_t)256 << 20;
  while (chunk > 1 && chunk * vocab * es > cap) chunk = (chunk + 1) / 2;
  const size_t lbytes = ((chunk * vocab * es + 255) / 256) * 256;
  const size_t rbytes = ((rows * 8 + 255) / 256) * 256 + 256;
  NML_TRY(g_scratch.ensure(lbytes + 2 * rbytes + 256));
  char* base = static_cast<char*>(g_scratch.p);
  void* logits = base;
  float* row_loss = reinterpret_cast<float*>(base + lbytes);
  int* row_valid = reinterpret_cast<int*>(base + lbytes + rbytes);
  double* acc = reinterpret_cast<double*>(base + lbytes + 2 * rbytes);
  int* err = reinterpret_cast<int*>(acc + 3);
  hipStream_t st = nml::stream();
  NML_HIP(hipMemsetAsync(err, 0, sizeof(int), st));
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
  if (rows == 0) NML_HIP(hipMemsetAsync(acc, 0, 2 * sizeof(double), st));
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
