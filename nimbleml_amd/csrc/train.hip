// Training on the device (float32 and float16 models): compute_loss keeping what the
// backward needs, then loss.backward() into a float32 gradient arena laid out like the
// parameter arena (one element per parameter element)
// (models/gpt.py:123-137 with the reference's autograd: losses/cross_entropy.py:109-192,
// kernels/fused_tied_crossentropy.py:27-48, neural_network/_fused_arrays.py:129-377,
// kernels/fused_rmsnorm.py:208-217, kernels/embedding_scatter.py:39-60).
//
// Saved per layer l over R = B·S rows: the block input X[l], N1 = RMSNorm₁(X[l]), q/k/v
// head-major (after RoPE), the merged attention output, the softmax log-sum-exp, the
// mid-block residual XM, N2 = RMSNorm₂(XM), the FFN pre-activation and GELU output; then
// X[L] and the final-normed H. The logits are not kept: the backward forms them again
// chunk by chunk (one more head GEMM instead of R·V floats).
//
// Backward, with G the gradient of the residual stream (R, d):
//   head:  dlogits = (softmax − onehot)·scale/n;  dH = dlogits·E;  dE += dlogitsᵀ·H
//   final: G = RMSNormᵀ(dH)
//   block: dW₂ += Gᵀ·hid, db₂ += Σ G, dpre = (G·W₂)∘gelu'(pre), dW₁ += dpreᵀ·N2,
//          db₁ += Σ dpre, G += RMSNorm₂ᵀ(dpre·W₁);
//          dW_o += Gᵀ·att, db_o += Σ G, datt = G·W_o → attention backward → dqkv
//          (RoPE inverse on dq, dk), dW_qkv += dqkvᵀ·N1, db_qkv += Σ dqkv,
//          G += RMSNorm₁ᵀ(dqkv·W_qkv)
//   embeddings: dE[ids] += G, dpos[s] += Σ_b G
// Weight gradients are (out, in) like the device weights.
#include <cstring>

#include "model.hpp"

namespace nml {

struct TrainState {
  Buf grads;    // float32, one element per parameter element, the parameter arena's layout
  Buf moments;  // AdamW first and second moments, two more float32 arenas of that layout
  Buf masters;  // fp16 models: float32 master copies of the parameters (optimizers/adam.py:75-81)
  Buf acts;     // saved activations of the last loss_train
  Buf scratch;  // backward scratch
  Buf io;       // ids and labels of the last loss_train, loss accumulators
  Buf mask;     // the (S, S) additive mask of a saved module forward, when it took one
  int B = 0, S = 0;
  bool saved = false;
  int what = 0;        // the saved forward: kSavedLoss, kSavedBlocks or kSavedMha
  int final_norm = 0;  // kSavedBlocks: the final RMSNorm ran after the blocks
  int full = 0;        // module forwards: non-causal attention
  int masked = 0;      // ... with the additive mask kept in `mask`
  int mha_layer = 0;   // kSavedMha: the layer whose attention ran
  unsigned long long generation = 0;  // advanced by every saving forward: which one is saved
  long long ignore_index = 0;
  int has_ignore = 0;
  double n_valid = 0.0;
};

constexpr int kSavedLoss = 1, kSavedBlocks = 2, kSavedMha = 3;

void train_release(nml_model* m) {
  if (!m->train) return;
  m->train->mask.release();
  m->train->grads.release();
  m->train->moments.release();
  m->train->masters.release();
  m->train->acts.release();
  m->train->scratch.release();
  m->train->io.release();
  delete m->train;
  m->train = nullptr;
}

namespace {

// Saved activations of R rows (storage type, es bytes each), carved from one buffer; the
// log-sum-exp rows are float32.
struct Saved {
  char *x, *n1, *q, *k, *v, *att, *xm, *n2, *pre, *hid;  // layer 0; + l·stride
  float* lse;
  size_t stride;  // bytes per layer
  char* xl;       // X[L]
  char* hf;       // final-normed
};

size_t saved_bytes(const nml_model* m, int B, int S, Saved* s, char* base) {
  const size_t R = (size_t)B * S, rd = align256(R * m->d * m->es), rf = align256(R * m->F * m->es);
  const size_t rl = align256((size_t)B * m->H * S * 4);
  const size_t per = 8 * rd + 2 * rf + rl;
  if (s) {
    char* p = base;
    s->x = p; p += rd;
    s->n1 = p; p += rd;
    s->q = p; p += rd;
    s->k = p; p += rd;
    s->v = p; p += rd;
    s->att = p; p += rd;
    s->xm = p; p += rd;
    s->n2 = p; p += rd;
    s->pre = p; p += rf;
    s->hid = p; p += rf;
    s->lse = reinterpret_cast<float*>(p);
    s->stride = per;
    s->xl = base + per * m->L;
    s->hf = s->xl + rd;
  }
  return per * m->L + 2 * rd;
}

inline char* at(char* p, const Saved& s, int l) { return p + s.stride * l; }
inline float* at(float* p, const Saved& s, int l) {
  return reinterpret_cast<float*>(reinterpret_cast<char*>(p) + s.stride * l);
}

// The float32 arenas hold one element per parameter element: parameter byte offset / es.
size_t f32_bytes(const nml_model* m) { return m->arena_bytes / m->es * 4; }
size_t f32_off(const nml_model* m, const void* param) {
  return static_cast<size_t>(static_cast<const char*>(param) - static_cast<const char*>(m->arena)) /
         m->es * 4;
}
float* grad_of(nml_model* m, const void* param) {
  return reinterpret_cast<float*>(static_cast<char*>(m->train->grads.p) + f32_off(m, param));
}

int ensure_train(nml_model* m) {
  if (!m->train) m->train = new TrainState();
  TrainState* t = m->train;
  if (!t->grads.p) {
    NML_TRY(t->grads.ensure(f32_bytes(m)));
    NML_HIP(hipMemsetAsync(t->grads.p, 0, f32_bytes(m), nml::stream()));
  }
  return 0;
}

// Rows per logits chunk: at most 512 MiB of logits at once.
size_t logits_chunk(const nml_model* m, size_t R) {
  size_t chunk = R;
  while (chunk > 1 && chunk * m->V * m->es > ((size_t)512 << 20)) chunk = (chunk + 1) / 2;
  return chunk;
}

LinearArgs lin(const void* x, long long lda, const void* w, const void* bias, void* out, int M,
               int N, int K, int epi, const void* resid = nullptr) {
  LinearArgs a{};
  a.x = x;
  a.lda = lda;
  a.w = w;
  a.bias = bias;
  a.out = out;
  a.resid = resid;
  a.M = M;
  a.N = N;
  a.K = K;
  a.epi = epi;
  return a;
}

GemmBwdArgs gb(const void* a, long long lda, const void* b, long long ldb, void* c, long long ldc,
               int M, int N, int K, const void* aux = nullptr, long long ldaux = 0) {
  GemmBwdArgs g{};
  g.a = a;
  g.lda = lda;
  g.b = b;
  g.ldb = ldb;
  g.c = c;
  g.ldc = ldc;
  g.aux = aux;
  g.ldaux = ldaux;
  g.M = M;
  g.N = N;
  g.K = K;
  return g;
}

// Parameter element ranges of the arena around the rotary tables (buffers, not
// parameters): [first, second) pairs in elements.
void param_ranges(const nml_model* m, size_t (&r)[2][2]) {
  const size_t total = m->arena_bytes / m->es;
  const size_t lo = static_cast<size_t>(static_cast<char*>(m->rope_cos) - static_cast<char*>(m->arena)) / m->es;
  const size_t hi = (static_cast<size_t>(static_cast<char*>(m->rope_sin) - static_cast<char*>(m->arena)) +
                     align256(param_elems(m, NML_P_ROPE_SIN) * m->es)) / m->es;
  r[0][0] = 0;
  r[0][1] = lo;
  r[1][0] = hi;
  r[1][1] = total;
}

// The AdamW state: zero first and second moments and, for fp16 models, float32 masters
// taken from the parameters (optimizers/adam.py:64-81), allocated once.
int ensure_adam(nml_model* m) {
  NML_TRY(ensure_train(m));
  TrainState* t = m->train;
  hipStream_t st = nml::stream();
  const size_t fb = f32_bytes(m);
  if (!t->moments.p) {
    NML_TRY(t->moments.ensure(2 * fb));
    NML_HIP(hipMemsetAsync(t->moments.p, 0, 2 * fb, st));
  }
  if (m->dt == F16 && !t->masters.p) {
    NML_TRY(t->masters.ensure(fb));
    NML_TRY(launch_convert(F16, m->arena, F32, t->masters.p, m->arena_bytes / m->es, st));
  }
  return 0;
}

// What AdamW updates: the float32 parameters themselves, or the fp16 models' masters.
float* master_base(nml_model* m) {
  return static_cast<float*>(m->dt == F16 ? m->train->masters.p : m->arena);
}


// Attention of a saved forward: causal, or full (non-causal) with an optional (S, S)
// additive mask of the model's type.
struct MaskMode {
  int full = 0;
  const void* mask = nullptr;
};

// The attention half of a block over R = B·S rows of n1 (its normalised input):
// [q | k | v] = n1·W_qkvᵀ + b into head-major q, k, v, RoPE when `rope`, attention into att
// (merged heads) with each row's log-sum-exp in lse (_fused_arrays.py:52-104).
int attn_forward_saving(nml_model* m, const Layer& w, int B, int S, const char* n1, char* q,
                        char* k, char* v, char* att, float* lse, MaskMode mm, bool rope,
                        hipStream_t st) {
  const int R = B * S, d = m->d, dt = m->dt;
  const long long sb = (long long)m->H * S * m->dk, sh = (long long)S * m->dk;
  LinearArgs qkv = lin(n1, d, w.wqkv, w.bqkv, nullptr, R, 3 * d, d, EPI_QKV);
  qkv.qkv = QKVDst{q, k, v, nullptr, sb, sh, S, m->H, m->dk, d, nullptr};
  NML_TRY(launch_linear(dt, qkv, st));
  if (rope)
    NML_TRY(launch_rope(dt, q, k, sb, sh, B, m->H, S, m->dk, nullptr, nullptr, m->rope_cos,
                        m->rope_sin, m->P, st));
  AttnArgs a{};
  a.q = q;
  a.k = k;
  a.v = v;
  a.out = att;
  a.kv_stride_b = sb;
  a.kv_stride_h = sh;
  a.B = B;
  a.H = m->H;
  a.S = S;
  a.dk = m->dk;
  a.scale = sqrtf((float)m->dk);
  a.lse = lse;
  a.full = mm.full;
  a.mask = mm.mask;
  return launch_attention_prefill(dt, a, st);
}

// Every block over R = B·S rows of sv.x (layer 0's input), keeping what the backward
// reads; the last block's output lands in sv.xl (_fused_arrays.py:251-296).
int blocks_forward_saving(nml_model* m, const Saved& sv, int B, int S, MaskMode mm,
                          hipStream_t st) {
  const int R = B * S, d = m->d, F = m->F, dt = m->dt;
  for (int l = 0; l < m->L; ++l) {
    const Layer& w = m->layers[l];
    char *x = at(sv.x, sv, l), *n1 = at(sv.n1, sv, l), *q = at(sv.q, sv, l), *k = at(sv.k, sv, l),
         *v = at(sv.v, sv, l), *att = at(sv.att, sv, l), *xm = at(sv.xm, sv, l),
         *n2 = at(sv.n2, sv, l), *pre = at(sv.pre, sv, l), *hid = at(sv.hid, sv, l);
    float* lse = at(sv.lse, sv, l);
    char* xnext = l + 1 < m->L ? at(sv.x, sv, l + 1) : sv.xl;
    NML_TRY(launch_rmsnorm(dt, x, w.ln1, n1, nullptr, nullptr, R, d, kEps, st));
    NML_TRY(attn_forward_saving(m, w, B, S, n1, q, k, v, att, lse, mm, rope_on(m), st));
    NML_TRY(launch_linear(dt, lin(att, d, w.wo, w.bo, xm, R, d, d, EPI_BIAS_RESID, x), st));
    NML_TRY(launch_rmsnorm(dt, xm, w.ln2, n2, nullptr, nullptr, R, d, kEps, st));
    if (R > 64) {  // GELU in the GEMM's epilogue, which also keeps the pre-activation
      LinearArgs f1 = lin(n2, d, w.w1, w.b1, hid, R, F, d, EPI_BIAS_GELU);
      f1.pre_out = pre;
      NML_TRY(launch_linear(dt, f1, st));
    } else {
      NML_TRY(launch_linear(dt, lin(n2, d, w.w1, w.b1, pre, R, F, d, EPI_BIAS), st));
      NML_TRY(launch_gelu(dt, pre, hid, nullptr, (size_t)R * F, st));
    }
    NML_TRY(launch_linear(dt, lin(hid, F, w.w2, w.b2, xnext, R, d, F, EPI_BIAS_RESID, xm), st));
  }
  return 0;
}

// Backward scratch (storage type): G, DX (R, d); DQKV (R, 3d); DPRE (R, F); then float32
// DVEC (B, H, S) and the row- and column-sum partials.
struct BwdScratch {
  char *G, *DX, *DQKV, *DPRE;
  float *DVEC, *PART;
};

int bwd_scratch(nml_model* m, int B, int S, BwdScratch* w) {
  const int R = B * S, d = m->d, F = m->F;
  const size_t es = m->es;
  const size_t rd = align256((size_t)R * d * es), r3 = align256((size_t)R * 3 * d * es),
               rf = align256((size_t)R * F * es), rv = align256((size_t)B * m->H * S * 4);
  const int widest = F > 3 * d ? F : 3 * d;
  const size_t pn = (size_t)(rmsnorm_bwd_parts(R) > colsum_parts(R) ? rmsnorm_bwd_parts(R)
                                                                     : colsum_parts(R)) *
                    widest;
  NML_TRY(m->train->scratch.ensure(2 * rd + r3 + rf + rv + align256(pn * 4)));
  char* sp = static_cast<char*>(m->train->scratch.p);
  w->G = sp;
  w->DX = sp + rd;
  w->DQKV = sp + 2 * rd;
  w->DPRE = sp + 2 * rd + r3;
  w->DVEC = reinterpret_cast<float*>(sp + 2 * rd + r3 + rf);
  w->PART = reinterpret_cast<float*>(sp + 2 * rd + r3 + rf + rv);
  return 0;
}

// Backward of attn_forward_saving followed by its W_o projection, from ws.G = d/d(the
// projection's output): the W_o and W_qkv gradients are added to, ws.DX = d/d(n1)
// (_fused_arrays.py:129-184).
int attn_backward_saved(nml_model* m, const Layer& w, int B, int S, const char* n1,
                        const char* q, const char* k, const char* v, const char* att,
                        const float* lse, MaskMode mm, bool rope, const BwdScratch& ws,
                        hipStream_t st) {
  const int R = B * S, d = m->d, dt = m->dt;
  NML_TRY(launch_gemm_bwd(dt, gb(ws.G, d, att, d, grad_of(m, w.wo), d, d, d, R), false, false, GB_ADD, st));
  NML_TRY(launch_colsum(dt, ws.G, d, R, d, grad_of(m, w.bo), ws.PART, st));
  NML_TRY(launch_gemm_bwd(dt, gb(ws.G, d, w.wo, d, ws.DX, d, R, d, d), true, false, GB_SET, st));
  AttnBwdArgs ab{};
  ab.q = q;
  ab.k = k;
  ab.v = v;
  ab.o = att;
  ab.dout = ws.DX;
  ab.lse = lse;
  ab.dvec = ws.DVEC;
  ab.dqkv = ws.DQKV;
  ab.B = B;
  ab.H = m->H;
  ab.S = S;
  ab.dk = m->dk;
  ab.scale = sqrtf((float)m->dk);
  ab.full = mm.full;
  ab.mask = mm.mask;
  NML_TRY(launch_attention_backward(dt, ab, st));
  if (rope)
    NML_TRY(launch_rope_backward(dt, ws.DQKV, R, S, m->H, m->dk, m->rope_cos, m->rope_sin, st));
  NML_TRY(launch_gemm_bwd(dt, gb(ws.DQKV, 3 * d, n1, d, grad_of(m, w.wqkv), d, 3 * d, d, R), false,
                          false, GB_ADD, st));
  NML_TRY(launch_colsum(dt, ws.DQKV, 3 * d, R, 3 * d, grad_of(m, w.bqkv), ws.PART, st));
  return launch_gemm_bwd(dt, gb(ws.DQKV, 3 * d, w.wqkv, d, ws.DX, d, R, d, 3 * d), true, false,
                         GB_SET, st);
}

// Backward of blocks_forward_saving: ws.G holds d/d(sv.xl) on entry and d/d(layer 0's
// input) on return; every block parameter's gradient is added to
// (_fused_arrays.py:335-377, in reverse block order as :311-332 runs them).
int blocks_backward_saved(nml_model* m, const Saved& sv, int B, int S, MaskMode mm,
                          const BwdScratch& ws, hipStream_t st) {
  const int R = B * S, d = m->d, F = m->F, dt = m->dt;
  for (int l = m->L - 1; l >= 0; --l) {
    const Layer& w = m->layers[l];
    const char *x = at(sv.x, sv, l), *n1 = at(sv.n1, sv, l), *q = at(sv.q, sv, l),
               *k = at(sv.k, sv, l), *v = at(sv.v, sv, l), *att = at(sv.att, sv, l),
               *xm = at(sv.xm, sv, l), *n2 = at(sv.n2, sv, l), *pre = at(sv.pre, sv, l),
               *hid = at(sv.hid, sv, l);
    const float* lse = at(sv.lse, sv, l);
    // FFN (_fused_arrays.py:225-248)
    NML_TRY(launch_gemm_bwd(dt, gb(ws.G, d, hid, F, grad_of(m, w.w2), F, d, F, R), false, false, GB_ADD, st));
    NML_TRY(launch_colsum(dt, ws.G, d, R, d, grad_of(m, w.b2), ws.PART, st));
    NML_TRY(launch_gemm_bwd(dt, gb(ws.G, d, w.w2, F, ws.DPRE, F, R, F, d, pre, F), true, false, GB_GELU, st));
    NML_TRY(launch_gemm_bwd(dt, gb(ws.DPRE, F, n2, d, grad_of(m, w.w1), d, F, d, R), false, false, GB_ADD, st));
    NML_TRY(launch_colsum(dt, ws.DPRE, F, R, F, grad_of(m, w.b1), ws.PART, st));
    NML_TRY(launch_gemm_bwd(dt, gb(ws.DPRE, F, w.w1, d, ws.DX, d, R, d, F), true, false, GB_SET, st));
    NML_TRY(launch_rmsnorm_bwd(dt, ws.DX, xm, w.ln2, ws.G, 1, grad_of(m, w.ln2), ws.PART, R, d, kEps, st));
    // MHA (_fused_arrays.py:129-184), then RMSNorm₁ into the residual gradient
    NML_TRY(attn_backward_saved(m, w, B, S, n1, q, k, v, att, lse, mm, rope_on(m), ws, st));
    NML_TRY(launch_rmsnorm_bwd(dt, ws.DX, x, w.ln1, ws.G, 1, grad_of(m, w.ln1), ws.PART, R, d, kEps, st));
  }
  return 0;
}

// A module forward's mask mode; a mask is copied into the training state, since the
// backward reads it after the caller's buffer may be gone.
int module_mask(nml_model* m, int S, int causal, const void* mask, hipStream_t st, MaskMode* mm) {
  TrainState* t = m->train;
  mm->full = causal ? 0 : 1;
  mm->mask = nullptr;
  t->full = mm->full;
  t->masked = mask != nullptr;
  if (mask && S > 0) {
    const size_t bytes = (size_t)S * S * m->es;
    NML_TRY(t->mask.ensure(bytes));
    NML_HIP(hipMemcpyAsync(t->mask.p, mask, bytes, hipMemcpyDeviceToDevice, st));
    mm->mask = t->mask.p;
  }
  return 0;
}

MaskMode saved_mask(const TrainState* t) {
  MaskMode mm;
  mm.full = t->full;
  mm.mask = t->masked ? t->mask.p : nullptr;
  return mm;
}

}  // namespace

int train_param_uploaded(nml_model* m, const void* param, size_t elems) {
  if (m->dt != F16 || !m->train || !m->train->masters.p) return 0;
  return launch_convert(F16, param, F32, static_cast<char*>(m->train->masters.p) + f32_off(m, param),
                        elems, nml::stream());
}

}  // namespace nml

using namespace nml;

extern "C" {

int nml_model_zero_grad(nml_model* m) {
  NML_TRY(check_ready(m));
  NML_TRY(ensure_train(m));
  NML_HIP(hipMemsetAsync(m->train->grads.p, 0, f32_bytes(m), nml::stream()));
  NML_HIP(hipStreamSynchronize(nml::stream()));
  return 0;
}

int nml_model_grad_ptr(nml_model* m, int kind, int layer, void** ptr) {
  NML_TRY(check_ready(m));
  NML_REQUIRE(kind != NML_P_ROPE_COS && kind != NML_P_ROPE_SIN,
              "rotary tables are buffers, not parameters: no gradient");
  void** slot = param_slot(m, kind, layer);
  NML_REQUIRE(slot != nullptr, "unknown parameter kind %d / layer %d", kind, layer);
  NML_TRY(ensure_train(m));
  *ptr = grad_of(m, *slot);
  return 0;
}

int nml_model_loss_train(nml_model* m, const int64_t* ids, const int64_t* labels, size_t batch,
                         size_t seq, int64_t ignore_index, int has_ignore, double* loss) {
  NML_TRY(check_ready(m));
  NML_REQUIRE(seq <= (size_t)m->P, "Sequence length %zu exceeds maximum sequence length %d", seq,
              m->P);
  NML_TRY(ensure_train(m));
  TrainState* t = m->train;
  t->saved = false;
  const int B = (int)batch, S = (int)seq, R = B * S, d = m->d, dt = m->dt;
  const size_t es = m->es;
  if (R == 0) {
    *loss = 0.0;
    return 0;
  }
  hipStream_t st = nml::stream();
  Saved sv;
  NML_TRY(t->acts.ensure(saved_bytes(m, B, S, nullptr, nullptr)));
  saved_bytes(m, B, S, &sv, static_cast<char*>(t->acts.p));
  // io: ids, labels, then err / loss accumulators, per-row loss and validity
  const size_t ib = align256((size_t)R * 8), rb = align256((size_t)R * 4);
  NML_TRY(t->io.ensure(2 * ib + 512 + 2 * rb));
  char* io = static_cast<char*>(t->io.p);
  int64_t* dids = reinterpret_cast<int64_t*>(io);
  int64_t* dlab = reinterpret_cast<int64_t*>(io + ib);
  int* err = reinterpret_cast<int*>(io + 2 * ib);
  double* acc = reinterpret_cast<double*>(io + 2 * ib + 256);
  float* row_loss = reinterpret_cast<float*>(io + 2 * ib + 512);
  int* row_valid = reinterpret_cast<int*>(io + 2 * ib + 512 + rb);
  NML_HIP(hipMemcpyAsync(dids, ids, (size_t)R * 8, hipMemcpyDeviceToDevice, st));
  NML_HIP(hipMemcpyAsync(dlab, labels, (size_t)R * 8, hipMemcpyDeviceToDevice, st));
  NML_HIP(hipMemsetAsync(err, 0, sizeof(int), st));

  NML_TRY(launch_embed(dt, dids, m->emb, posw(m), nullptr, sv.x, B, S, d, m->V, m->P, err, st));
  NML_TRY(blocks_forward_saving(m, sv, B, S, MaskMode{}, st));
  NML_TRY(launch_rmsnorm(dt, sv.xl, m->lnf, sv.hf, nullptr, nullptr, R, d, kEps, st));

  const size_t chunk = logits_chunk(m, R);
  NML_TRY(m->logits_ws.ensure(align256(chunk * m->V * es)));
  for (size_t r0 = 0; r0 < (size_t)R; r0 += chunk) {
    const int n = (int)(((size_t)R - r0 < chunk) ? (size_t)R - r0 : chunk);
    NML_TRY(launch_linear(dt, lin(sv.hf + r0 * d * es, d, m->emb, nullptr, m->logits_ws.p, n, m->V,
                                  d, EPI_NONE), st));
    NML_TRY(launch_ce_rows(dt, m->logits_ws.p, n, m->V, dlab + r0, ignore_index, has_ignore,
                           row_loss, row_valid, err, st));
    NML_TRY(launch_ce_reduce(row_loss, row_valid, n, acc, r0 > 0, st));
  }
  NML_TRY(launch_ce_finalize(acc, acc + 2, st));
  double host[3];
  int herr = 0;
  NML_HIP(hipMemcpyAsync(host, acc, sizeof(host), hipMemcpyDeviceToHost, st));
  NML_HIP(hipMemcpyAsync(&herr, err, sizeof(int), hipMemcpyDeviceToHost, st));
  NML_HIP(hipStreamSynchronize(st));
  NML_REQUIRE((herr & 1) == 0, "Token ID out of range [0, %d)", m->V);
  NML_REQUIRE((herr & 2) == 0, "label out of range [0, %d)", m->V);
  *loss = host[2];
  t->B = B;
  t->S = S;
  t->ignore_index = ignore_index;
  t->has_ignore = has_ignore;
  t->n_valid = host[1];
  t->what = kSavedLoss;
  t->saved = true;
  t->generation += 1;
  return 0;
}

int nml_model_backward(nml_model* m, double grad_scale) {
  NML_TRY(check_ready(m));
  NML_REQUIRE(m->train && m->train->saved && m->train->what == kSavedLoss,
              "backward: no saved loss forward (call nml_model_loss_train first)");
  TrainState* t = m->train;
  const int B = t->B, S = t->S, R = B * S, d = m->d, V = m->V, dt = m->dt;
  const size_t es = m->es;
  if (t->n_valid <= 0.0) return 0;  // every label ignored: the loss is a constant 0
  hipStream_t st = nml::stream();
  Saved sv;
  saved_bytes(m, B, S, &sv, static_cast<char*>(t->acts.p));
  const size_t ib = align256((size_t)R * 8);
  const int64_t* dids = reinterpret_cast<const int64_t*>(t->io.p);
  const int64_t* dlab = reinterpret_cast<const int64_t*>(static_cast<char*>(t->io.p) + ib);

  BwdScratch ws;
  NML_TRY(bwd_scratch(m, B, S, &ws));
  char* G = ws.G;
  char* DX = ws.DX;
  float* PART = ws.PART;
  const void* E = m->emb;
  float* dE = grad_of(m, m->emb);

  // tied head + cross-entropy, chunk by chunk; dH lands in DX
  const float scale = static_cast<float>(grad_scale / t->n_valid);
  const size_t chunk = logits_chunk(m, R);
  NML_TRY(m->logits_ws.ensure(align256(chunk * V * es)));
  void* lg = m->logits_ws.p;
  for (size_t r0 = 0; r0 < (size_t)R; r0 += chunk) {
    const int n = (int)(((size_t)R - r0 < chunk) ? (size_t)R - r0 : chunk);
    const char* h = sv.hf + r0 * d * es;
    NML_TRY(launch_linear(dt, lin(h, d, E, nullptr, lg, n, V, d, EPI_NONE), st));
    NML_TRY(launch_ce_grad(dt, lg, n, V, dlab + r0, t->ignore_index, t->has_ignore, scale, st));
    NML_TRY(launch_gemm_bwd(dt, gb(lg, V, E, d, DX + r0 * d * es, d, n, d, V), true, false, GB_SET, st));
    NML_TRY(launch_gemm_bwd(dt, gb(lg, V, h, d, dE, d, V, d, n), false, false, GB_ADD, st));
  }
  NML_TRY(launch_rmsnorm_bwd(dt, DX, sv.xl, m->lnf, G, 0, grad_of(m, m->lnf), PART, R, d, kEps, st));

  NML_TRY(blocks_backward_saved(m, sv, B, S, MaskMode{}, ws, st));
  NML_TRY(launch_embed_backward(dt, G, dids, dE, rope_on(m) ? nullptr : grad_of(m, m->pos), B, S, d,
                                V, st));
  NML_HIP(hipStreamSynchronize(st));
  return 0;
}

int nml_model_logits_backward(nml_model* m, const int64_t* ids, size_t batch, size_t seq,
                              const void* dlogits) {
  NML_TRY(check_ready(m));
  NML_REQUIRE(seq <= (size_t)m->P, "Sequence length %zu exceeds maximum sequence length %d", seq,
              m->P);
  NML_TRY(ensure_train(m));
  TrainState* t = m->train;
  // the recompute below overwrites the saved activations of any earlier saving forward
  t->saved = false;
  t->generation += 1;
  const int B = (int)batch, S = (int)seq, R = B * S, d = m->d, V = m->V, dt = m->dt;
  if (R == 0) return 0;
  hipStream_t st = nml::stream();
  Saved sv;
  NML_TRY(t->acts.ensure(saved_bytes(m, B, S, nullptr, nullptr)));
  saved_bytes(m, B, S, &sv, static_cast<char*>(t->acts.p));
  const size_t ib = align256((size_t)R * 8);
  NML_TRY(t->io.ensure(ib + 256));
  int64_t* dids = reinterpret_cast<int64_t*>(t->io.p);
  int* err = reinterpret_cast<int*>(static_cast<char*>(t->io.p) + ib);
  NML_HIP(hipMemcpyAsync(dids, ids, (size_t)R * 8, hipMemcpyDeviceToDevice, st));
  NML_HIP(hipMemsetAsync(err, 0, sizeof(int), st));
  // the forward of GPT.forward, keeping what the backward reads
  NML_TRY(launch_embed(dt, dids, m->emb, posw(m), nullptr, sv.x, B, S, d, V, m->P, err, st));
  NML_TRY(blocks_forward_saving(m, sv, B, S, MaskMode{}, st));
  NML_TRY(launch_rmsnorm(dt, sv.xl, m->lnf, sv.hf, nullptr, nullptr, R, d, kEps, st));
  BwdScratch ws;
  NML_TRY(bwd_scratch(m, B, S, &ws));
  // tied head (gpt.py:150-153): dH = dlogits·E, dE += dlogitsᵀ·H
  float* dE = grad_of(m, m->emb);
  NML_TRY(launch_gemm_bwd(dt, gb(dlogits, V, m->emb, d, ws.DX, d, R, d, V), true, false, GB_SET, st));
  NML_TRY(launch_gemm_bwd(dt, gb(dlogits, V, sv.hf, d, dE, d, V, d, R), false, false, GB_ADD, st));
  NML_TRY(launch_rmsnorm_bwd(dt, ws.DX, sv.xl, m->lnf, ws.G, 0, grad_of(m, m->lnf), ws.PART, R, d,
                             kEps, st));
  NML_TRY(blocks_backward_saved(m, sv, B, S, MaskMode{}, ws, st));
  NML_TRY(launch_embed_backward(dt, ws.G, dids, dE, rope_on(m) ? nullptr : grad_of(m, m->pos), B,
                                S, d, V, st));
  int herr = 0;
  NML_HIP(hipMemcpyAsync(&herr, err, sizeof(int), hipMemcpyDeviceToHost, st));
  NML_HIP(hipStreamSynchronize(st));
  NML_REQUIRE((herr & 1) == 0, "Token ID out of range [0, %d)", V);
  return 0;
}

// ------------------------------------------------------------ module-level autograd
// A saving forward of a module: shape checks, the activation buffer carved, the mask kept.
static int module_forward_begin(nml_model* m, size_t batch, size_t seq, int causal,
                                const void* mask, const char* what, Saved* sv, MaskMode* mm) {
  NML_REQUIRE(m != nullptr, "model is null");
  NML_REQUIRE(seq <= (size_t)m->P, "Sequence length %zu exceeds maximum sequence length %d", seq,
              m->P);
  NML_REQUIRE(!causal || mask == nullptr, "%s: a causal call takes no mask", what);
  NML_TRY(ensure_train(m));
  TrainState* t = m->train;
  t->saved = false;
  const int B = (int)batch, S = (int)seq;
  NML_TRY(t->acts.ensure(saved_bytes(m, B, S, nullptr, nullptr)));
  saved_bytes(m, B, S, sv, static_cast<char*>(t->acts.p));
  NML_TRY(module_mask(m, S, causal, mask, nml::stream(), mm));
  t->B = B;
  t->S = S;
  return 0;
}

static void module_forward_end(nml_model* m, int what) {
  m->train->what = what;
  m->train->saved = true;
  m->train->generation += 1;
}

static int module_backward_begin(nml_model* m, int what, const char* name, Saved* sv,
                                 BwdScratch* ws) {
  NML_REQUIRE(m != nullptr, "model is null");
  NML_REQUIRE(m->train && m->train->saved && m->train->what == what,
              "%s: no saved forward of this kind (run its saving forward first)", name);
  TrainState* t = m->train;
  saved_bytes(m, t->B, t->S, sv, static_cast<char*>(t->acts.p));
  if (t->B * t->S == 0) return 0;
  return bwd_scratch(m, t->B, t->S, ws);
}

int nml_model_blocks_forward_train(nml_model* m, const void* x, void* out, size_t batch,
                                   size_t seq, int final_norm, int causal, const void* mask) {
  Saved sv;
  MaskMode mm;
  NML_TRY(module_forward_begin(m, batch, seq, causal, mask, "blocks_forward_train", &sv, &mm));
  const int B = (int)batch, S = (int)seq, R = B * S;
  m->train->final_norm = final_norm != 0;
  if (R > 0) {
    hipStream_t st = nml::stream();
    const size_t bytes = (size_t)R * m->d * m->es;
    NML_HIP(hipMemcpyAsync(sv.x, x, bytes, hipMemcpyDeviceToDevice, st));
    NML_TRY(blocks_forward_saving(m, sv, B, S, mm, st));
    if (final_norm)
      NML_TRY(launch_rmsnorm(m->dt, sv.xl, m->lnf, sv.hf, nullptr, nullptr, R, m->d, kEps, st));
    NML_HIP(hipMemcpyAsync(out, final_norm ? sv.hf : sv.xl, bytes, hipMemcpyDeviceToDevice, st));
  }
  module_forward_end(m, kSavedBlocks);
  return 0;
}

int nml_model_blocks_backward(nml_model* m, const void* dout, void* dx) {
  Saved sv;
  BwdScratch ws;
  NML_TRY(module_backward_begin(m, kSavedBlocks, "blocks_backward", &sv, &ws));
  TrainState* t = m->train;
  const int B = t->B, S = t->S, R = B * S, d = m->d;
  if (R == 0) return 0;
  hipStream_t st = nml::stream();
  const size_t bytes = (size_t)R * d * m->es;
  if (t->final_norm)  // fused_trunk_backward_arrays (_fused_arrays.py:311-332): final norm first
    NML_TRY(launch_rmsnorm_bwd(m->dt, dout, sv.xl, m->lnf, ws.G, 0, grad_of(m, m->lnf), ws.PART,
                               R, d, kEps, st));
  else
    NML_HIP(hipMemcpyAsync(ws.G, dout, bytes, hipMemcpyDeviceToDevice, st));
  NML_TRY(blocks_backward_saved(m, sv, B, S, saved_mask(t), ws, st));
  if (dx) NML_HIP(hipMemcpyAsync(dx, ws.G, bytes, hipMemcpyDeviceToDevice, st));
  NML_HIP(hipStreamSynchronize(st));
  return 0;
}

int nml_model_mha_forward_train(nml_model* m, int layer, const void* x, void* out, size_t batch,
                                size_t seq, int causal, const void* mask) {
  NML_REQUIRE(m != nullptr, "model is null");
  NML_REQUIRE(layer >= 0 && layer < m->L, "layer %d outside [0, %d)", layer, m->L);
  Saved sv;
  MaskMode mm;
  NML_TRY(module_forward_begin(m, batch, seq, causal, mask, "mha_forward_train", &sv, &mm));
  const int B = (int)batch, S = (int)seq, R = B * S, d = m->d;
  m->train->mha_layer = layer;
  if (R > 0) {
    // the layer-0 slots of the saved buffer: n1 holds the input, then q, k, v, att, lse
    hipStream_t st = nml::stream();
    const Layer& w = m->layers[layer];
    NML_HIP(hipMemcpyAsync(sv.n1, x, (size_t)R * d * m->es, hipMemcpyDeviceToDevice, st));
    // neural_network/attention.py:139-168 applies no rotary embedding
    NML_TRY(attn_forward_saving(m, w, B, S, sv.n1, sv.q, sv.k, sv.v, sv.att, sv.lse, mm, false,
                                st));
    NML_TRY(launch_linear(m->dt, lin(sv.att, d, w.wo, w.bo, out, R, d, d, EPI_BIAS), st));
  }
  module_forward_end(m, kSavedMha);
  return 0;
}

int nml_model_mha_backward(nml_model* m, const void* dout, void* dx) {
  Saved sv;
  BwdScratch ws;
  NML_TRY(module_backward_begin(m, kSavedMha, "mha_backward", &sv, &ws));
  TrainState* t = m->train;
  const int B = t->B, S = t->S, R = B * S;
  if (R == 0) return 0;
  hipStream_t st = nml::stream();
  const size_t bytes = (size_t)R * m->d * m->es;
  NML_HIP(hipMemcpyAsync(ws.G, dout, bytes, hipMemcpyDeviceToDevice, st));
  NML_TRY(attn_backward_saved(m, m->layers[t->mha_layer], B, S, sv.n1, sv.q, sv.k, sv.v, sv.att,
                              sv.lse, saved_mask(t), false, ws, st));
  if (dx) NML_HIP(hipMemcpyAsync(dx, ws.DX, bytes, hipMemcpyDeviceToDevice, st));
  NML_HIP(hipStreamSynchronize(st));
  return 0;
}

int nml_model_adam_state_init(nml_model* m) {
  NML_TRY(check_ready(m));
  return ensure_adam(m);
}

int nml_model_adamw_step(nml_model* m, float lr, float beta1, float beta2, float bias_corr1,
                         float bias_corr2, float eps, float weight_decay) {
  NML_TRY(check_ready(m));
  NML_TRY(ensure_adam(m));
  TrainState* t = m->train;
  hipStream_t st = nml::stream();
  const size_t n_all = m->arena_bytes / m->es;
  // float32 parameters are updated in place; fp16 ones through their float32 masters,
  // the parameters rounded from the updated masters in the same pass (adam.py:238-245)
  float* master = master_base(m);
  size_t ranges[2][2];
  param_ranges(m, ranges);
  float* g = static_cast<float*>(t->grads.p);
  float* mm = static_cast<float*>(t->moments.p);
  for (const auto& r : ranges) {
    if (r[1] <= r[0]) continue;
    NML_TRY(launch_adamw(master + r[0], g + r[0], mm + r[0], mm + n_all + r[0], r[1] - r[0], lr,
                         beta1, beta2, bias_corr1, bias_corr2, eps, weight_decay, st,
                         m->dt == F16 ? static_cast<char*>(m->arena) + r[0] * m->es : nullptr));
  }
  return 0;
}

int nml_model_adamw_update(nml_model* m, int kind, int layer, size_t offset, size_t count,
                           float lr, float beta1, float beta2, float bias_corr1, float bias_corr2,
                           float eps, float weight_decay) {
  NML_TRY(check_ready(m));
  NML_REQUIRE(kind != NML_P_ROPE_COS && kind != NML_P_ROPE_SIN,
              "rotary tables are buffers, not parameters: no optimizer step");
  void** slot = param_slot(m, kind, layer);
  NML_REQUIRE(slot != nullptr, "unknown parameter kind %d / layer %d", kind, layer);
  NML_REQUIRE(offset <= param_elems(m, kind) && count <= param_elems(m, kind) - offset,
              "adamw_update: elements [%zu, %zu) outside parameter kind %d (%zu elements)", offset,
              offset + count, kind, param_elems(m, kind));
  NML_REQUIRE(offset % 4 == 0, "adamw_update: offset %zu must be a multiple of 4", offset);
  NML_TRY(ensure_adam(m));
  TrainState* t = m->train;
  const size_t n_all = m->arena_bytes / m->es;
  const size_t e0 = f32_off(m, *slot) / 4 + offset;  // element index in the arena
  float* mm = static_cast<float*>(t->moments.p);
  return launch_adamw(master_base(m) + e0, static_cast<float*>(t->grads.p) + e0, mm + e0,
                      mm + n_all + e0, count, lr, beta1, beta2, bias_corr1, bias_corr2, eps,
                      weight_decay, nml::stream(),
                      m->dt == F16 ? static_cast<char*>(m->arena) + e0 * m->es : nullptr);
}

int nml_model_adam_master(nml_model* m, int kind, int layer, void** master) {
  NML_TRY(check_ready(m));
  NML_REQUIRE(m->dt == F16, "float32 models keep no master copies (the parameters are updated)");
  NML_REQUIRE(kind != NML_P_ROPE_COS && kind != NML_P_ROPE_SIN,
              "rotary tables are buffers, not parameters: no master copy");
  void** slot = param_slot(m, kind, layer);
  NML_REQUIRE(slot != nullptr, "unknown parameter kind %d / layer %d", kind, layer);
  NML_REQUIRE(m->train && m->train->masters.p,
              "no optimizer state yet (call nml_model_adam_state_init)");
  *master = static_cast<char*>(m->train->masters.p) + f32_off(m, *slot);
  return 0;
}

int nml_model_adam_moments(nml_model* m, int kind, int layer, void** first, void** second) {
  NML_TRY(check_ready(m));
  NML_REQUIRE(kind != NML_P_ROPE_COS && kind != NML_P_ROPE_SIN,
              "rotary tables are buffers, not parameters: no optimizer state");
  void** slot = param_slot(m, kind, layer);
  NML_REQUIRE(slot != nullptr, "unknown parameter kind %d / layer %d", kind, layer);
  NML_REQUIRE(m->train && m->train->moments.p,
              "no optimizer state yet (call nml_model_adam_state_init or nml_model_adamw_step)");
  const size_t off = f32_off(m, *slot);
  *first = static_cast<char*>(m->train->moments.p) + off;
  *second = static_cast<char*>(m->train->moments.p) + f32_bytes(m) + off;
  return 0;
}

int nml_model_saved_generation(nml_model* m, unsigned long long* generation) {
  NML_REQUIRE(m != nullptr && generation != nullptr, "saved_generation: null argument");
  *generation = (m->train && m->train->saved) ? m->train->generation : 0;
  return 0;
}

}  // extern "C"
