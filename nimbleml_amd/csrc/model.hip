// GPT driver: device-resident parameters, the forward pass, compute_loss, the KV
// cache and the whole generate() loop (models/gpt.py, models/generate.py,
// neural_network/_fused_arrays.py:251-284 for the block).
//
// Per block, with x the residual stream (T) updated in place:
//   xn = RMSNorm₁(x);  [q | k | v] = xn·W_qkvᵀ + b   (q head-major; k, v into the cache)
//   a  = causal attention(q, K[0..pos], V[0..pos])  (merged heads)
//   x  = x + (a·W_oᵀ + b_o);  xn = RMSNorm₂(x)
//   h  = GELU(xn·W₁ᵀ + b₁);   x = x + (h·W₂ᵀ + b₂)
// then xn = RMSNorm_f(x) and logits = xn·Eᵀ (tied head).
#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "model.hpp"

using namespace nml;

struct nml_cache {
  nml_model* m;
  int B;
  void* k = nullptr;  // L × B × H × P × dk
  void* v = nullptr;
  int32_t* len_dev = nullptr;  // B
  std::vector<int32_t> len;    // host mirror
  // Single-token steps (forward_with_cache with one token per row): the fed ids at their
  // positions (B × P int64, row b at b·P) and the step's error word. Allocated on the
  // first such step.
  int64_t* tok = nullptr;
  int* err = nullptr;
};

namespace nml {

size_t param_elems(const nml_model* m, int kind) {
  const size_t d = m->d, F = m->F;
  switch (kind) {
    case NML_P_TOKEN_EMB: return (size_t)m->V * d;
    case NML_P_POS_EMB: return (size_t)m->P * d;
    case NML_P_ROPE_COS:
    case NML_P_ROPE_SIN: return (size_t)m->P * (m->dk / 2);
    case NML_P_LN_F:
    case NML_P_LN1:
    case NML_P_LN2:
    case NML_P_BO:
    case NML_P_B2: return d;
    case NML_P_WQKV: return 3 * d * d;
    case NML_P_BQKV: return 3 * d;
    case NML_P_WO: return d * d;
    case NML_P_W1: return F * d;
    case NML_P_B1: return F;
    case NML_P_W2: return d * F;
  }
  return 0;
}

void** param_slot(nml_model* m, int kind, int layer) {
  switch (kind) {
    case NML_P_TOKEN_EMB: return &m->emb;
    case NML_P_POS_EMB: return &m->pos;
    case NML_P_LN_F: return &m->lnf;
    case NML_P_ROPE_COS: return &m->rope_cos;
    case NML_P_ROPE_SIN: return &m->rope_sin;
  }
  if (layer < 0 || layer >= m->L) return nullptr;
  Layer& l = m->layers[layer];
  switch (kind) {
    case NML_P_LN1: return &l.ln1;
    case NML_P_WQKV: return &l.wqkv;
    case NML_P_BQKV: return &l.bqkv;
    case NML_P_WO: return &l.wo;
    case NML_P_BO: return &l.bo;
    case NML_P_LN2: return &l.ln2;
    case NML_P_W1: return &l.w1;
    case NML_P_B1: return &l.b1;
    case NML_P_W2: return &l.w2;
    case NML_P_B2: return &l.b2;
  }
  return nullptr;
}

const int kLayerKinds[10] = {NML_P_LN1, NML_P_WQKV, NML_P_BQKV, NML_P_WO, NML_P_BO,
                             NML_P_LN2, NML_P_W1,   NML_P_B1,   NML_P_W2, NML_P_B2};

int check_ready(nml_model* m) {
  NML_REQUIRE(m != nullptr, "model is null");
  NML_REQUIRE(m->emb && m->pos && m->lnf, "model parameters not uploaded");
  return 0;
}

}  // namespace nml

namespace {

// Activation workspace for R rows (B·S) of one forward.
struct Acts {
  void* x;   // (R, d) residual stream
  void* xn;  // (R, d) normalised
  void* q;   // (R, d) head-major queries
  void* att; // (R, d) merged attention output
  void* h;   // (R, F) FFN hidden
  void* part;   // decode attention workspace (zeroed before a decode loop)
  float* ssq;   // decode: (Bdec, d/16) sums of squares of x in 16-column pieces
};

int acts_in(nml_model* m, Buf& buf, int R, int Bdec, Acts* a) {
  const size_t rd = align256((size_t)R * m->d * m->es);
  const size_t rf = align256((size_t)R * m->F * m->es);
  const size_t part = Bdec ? align256(attention_decode_workspace(Bdec, m->H, m->dk, m->P)) : 0;
  const size_t ssq = Bdec ? align256((size_t)Bdec * (m->d / 16 + 1) * sizeof(float)) : 0;
  NML_TRY(buf.ensure(4 * rd + rf + part + ssq));
  char* b = static_cast<char*>(buf.p);
  a->x = b;
  a->xn = b + rd;
  a->q = b + 2 * rd;
  a->att = b + 3 * rd;
  a->h = b + 4 * rd;
  a->part = part ? static_cast<void*>(b + 4 * rd + rf) : nullptr;
  a->ssq = ssq ? reinterpret_cast<float*>(b + 4 * rd + rf + part) : nullptr;
  return 0;
}

int acts_for(nml_model* m, int R, int Bdec, Acts* a) { return acts_in(m, m->ws, R, Bdec, a); }

// Small device scratch: [0] int err, then B int32 positions etc.
struct Small {
  int* err;
  double* acc;   // 3 doubles
  int32_t* pos;  // up to 4096 rows
  int32_t* plen;
  int32_t* zeros;
};

int small_for(nml_model* m, int B, Small* s) {
  const size_t need = 256 + 256 + 3 * align256((size_t)B * 4 + 4);
  NML_TRY(m->small.ensure(need < 4096 ? 4096 : need));
  char* b = static_cast<char*>(m->small.p);
  s->err = reinterpret_cast<int*>(b);
  s->acc = reinterpret_cast<double*>(b + 256);
  const size_t bb = align256((size_t)B * 4 + 4);
  s->pos = reinterpret_cast<int32_t*>(b + 512);
  s->plen = reinterpret_cast<int32_t*>(b + 512 + bb);
  s->zeros = reinterpret_cast<int32_t*>(b + 512 + 2 * bb);
  return 0;
}

// Where a layer's K/V go: base pointers and strides.
struct KVView {
  void* k;
  void* v;
  long long sb, sh;
};

// Sequences of different lengths packed row after row (device arrays): row r is
// position s of sequence b with row_seg[r] = (b << 16) | s; sequence b has seq_len[b]
// rows starting at row_start[b]; R rows in all.
struct Ragged {
  const int32_t* row_seg;
  const int32_t* seq_len;
  const int32_t* row_start;
  int R;
};

// How a forward masks its attention: causal (the GPT path), or every key of a dense
// sequence plus an optional additive (S, S) mask (full != 0).
struct AttnMode {
  int full = 0;
  const void* mask = nullptr;
};

// One attention sublayer over R rows of xin: [q | k | v] = xin·W_qkvᵀ + b (q head-major
// into acts.q, k and v through c), RoPE when `rope`, attention into acts.att, then
// out = acts.att·W_oᵀ + b_o (+ resid when non-null; out may equal resid).
int attention_sublayer(nml_model* m, const Layer& w, const void* xin, const Acts& a, int B, int S,
                       const int32_t* pos_base, const KVView& c, bool rope, const AttnMode& am,
                       const void* resid, void* out, hipStream_t st, const Ragged* rg) {
  const int R = rg ? rg->R : B * S, d = m->d;
  LinearArgs qkv{};
  qkv.x = xin;
  qkv.lda = d;
  qkv.w = w.wqkv;
  qkv.bias = w.bqkv;
  qkv.M = R;
  qkv.N = 3 * d;
  qkv.K = d;
  qkv.epi = EPI_QKV;
  qkv.qkv = QKVDst{a.q, c.k, c.v, pos_base, c.sb, c.sh, S, m->H, m->dk, d,
                   rg ? rg->row_seg : nullptr};
  NML_TRY(launch_linear(m->dt, qkv, st));
  if (rope)  // models/gpt.py:62-64 → _fused_arrays.py:95-98
    NML_TRY(launch_rope(m->dt, a.q, c.k, c.sb, c.sh, B, m->H, S, m->dk, pos_base,
                        rg ? rg->seq_len : nullptr, m->rope_cos, m->rope_sin, m->P, st));
  AttnArgs at{};
  at.q = a.q;
  at.k = c.k;
  at.v = c.v;
  at.out = a.att;
  at.pos_base = pos_base;
  at.kv_stride_b = c.sb;
  at.kv_stride_h = c.sh;
  at.B = B;
  at.H = m->H;
  at.S = S;
  at.dk = m->dk;
  at.scale = sqrtf((float)m->dk);
  at.full = am.full;
  at.mask = am.mask;
  if (rg) {
    at.seq_len = rg->seq_len;
    at.row_start = rg->row_start;
  }
  NML_TRY(launch_attention_prefill(m->dt, at, st));
  LinearArgs wo{};
  wo.x = a.att;
  wo.lda = d;
  wo.w = w.wo;
  wo.bias = w.bo;
  wo.resid = resid;
  wo.out = out;
  wo.M = R;
  wo.N = d;
  wo.K = d;
  wo.epi = resid ? EPI_BIAS_RESID : EPI_BIAS;
  return launch_linear(m->dt, wo, st);
}

// The transformer trunk over R = B·S rows already embedded in acts.x (or rg->R packed
// ragged rows, S then being the longest length). Leaves the final-normed hidden states
// in acts.xn (final_norm) or the residual stream in acts.x (!final_norm: a stack of
// blocks without the trunk's last RMSNorm). pos_base (device, B) gives each row's first
// position (null → 0); kv(l) gives layer l's K/V destination.
template <typename KVF>
int trunk(nml_model* m, const Acts& a, int B, int S, const int32_t* pos_base, KVF kv,
          hipStream_t st, const Ragged* rg = nullptr, bool final_norm = true,
          const AttnMode& am = AttnMode{}) {
  const int R = rg ? rg->R : B * S, d = m->d;
  for (int l = 0; l < m->L; ++l) {
    const Layer& w = m->layers[l];
    const KVView c = kv(l);
    NML_TRY(launch_rmsnorm(m->dt, a.x, w.ln1, a.xn, nullptr, nullptr, R, d, kEps, st));
    NML_TRY(attention_sublayer(m, w, a.xn, a, B, S, pos_base, c, rope_on(m), am, a.x, a.x, st,
                               rg));
    NML_TRY(launch_rmsnorm(m->dt, a.x, w.ln2, a.xn, nullptr, nullptr, R, d, kEps, st));
    LinearArgs f1{};
    f1.x = a.xn;
    f1.lda = d;
    f1.w = w.w1;
    f1.bias = w.b1;
    f1.out = a.h;
    f1.M = R;
    f1.N = m->F;
    f1.K = d;
    f1.epi = EPI_BIAS_GELU;
    NML_TRY(launch_linear(m->dt, f1, st));
    LinearArgs f2{};
    f2.x = a.h;
    f2.lda = m->F;
    f2.w = w.w2;
    f2.bias = w.b2;
    f2.resid = a.x;
    f2.out = a.x;
    f2.M = R;
    f2.N = d;
    f2.K = m->F;
    f2.epi = EPI_BIAS_RESID;
    NML_TRY(launch_linear(m->dt, f2, st));
  }
  if (final_norm) NML_TRY(launch_rmsnorm(m->dt, a.x, m->lnf, a.xn, nullptr, nullptr, R, d, kEps, st));
  return 0;
}

// logits = xn · Eᵀ for all rows, or only the last position of each sequence.
int head(nml_model* m, const Acts& a, int B, int S, void* logits, int last_only, hipStream_t st) {
  LinearArgs lm{};
  lm.w = m->emb;
  lm.out = logits;
  lm.N = m->V;
  lm.K = m->d;
  lm.epi = EPI_NONE;
  if (last_only) {
    lm.x = static_cast<const char*>(a.xn) + (size_t)(S - 1) * m->d * m->es;
    lm.lda = (long long)S * m->d;
    lm.M = B;
  } else {
    lm.x = a.xn;
    lm.lda = m->d;
    lm.M = B * S;
  }
  return launch_linear(m->dt, lm, st);
}


// One decode step for rows [b0, b0 + Bn) of a cache: feeds tokens[b][pos[b]] at position
// pos[b], leaves those rows' logits (B, V; row b at b·V) in `logits`. tokens, pos and
// logits are the whole batch's arrays.
int decode_step(nml_model* m, nml_cache* c, const Acts& a, int b0, int Bn, const int64_t* tokens,
                long long tok_stride, int32_t* pos, int* err, void* logits, int max_len,
                hipStream_t st) {
  const int B = Bn, d = m->d;
  tokens += (long long)b0 * tok_stride;
  pos += b0;
  logits = static_cast<char*>(logits) + (size_t)b0 * m->V * m->es;
  NML_TRY(launch_embed_decode(m->dt, tokens, tok_stride, pos, m->emb, posw(m), a.x, B, d, m->V,
                              m->P, err, st));
  // the cache holds all c->B rows per layer; this step's rows start at row b0
  const size_t layer_kv = (size_t)c->B * m->H * m->P * m->dk * m->es;
  const size_t row0 = (size_t)b0 * m->H * m->P * m->dk * m->es;
  // RMSNorm fused into the GEMMs that consume it (fp16, 8 < B ≤ 64): the residual GEMMs
  // (W_o, W2) leave per-piece sums of squares of x in a.ssq, and QKV, W1 and the head
  // normalise x on load; layer 0's input (the embedding) still takes the RMSNorm kernel.
  const char* fuse_env = std::getenv("NIMBLEML_FUSE_NORM");  // "0": separate RMSNorm kernels
  const bool fuse = !(fuse_env && fuse_env[0] == '0') && a.ssq && linear_norm_fusable(m->dt, B, d, d) &&
                    linear_norm_fusable(m->dt, B, d, 3 * d) &&
                    linear_norm_fusable(m->dt, B, d, m->F) && linear_norm_fusable(m->dt, B, m->F, d) &&
                    linear_norm_fusable(m->dt, B, d, m->V);
  for (int l = 0; l < m->L; ++l) {
    const Layer& w = m->layers[l];
    void* kl = static_cast<char*>(c->k) + l * layer_kv + row0;
    void* vl = static_cast<char*>(c->v) + l * layer_kv + row0;
    const long long sb = (long long)m->H * m->P * m->dk, sh = (long long)m->P * m->dk;
    const bool fuse_in = fuse && l > 0;
    if (!fuse_in) NML_TRY(launch_rmsnorm(m->dt, a.x, w.ln1, a.xn, nullptr, nullptr, B, d, kEps, st));
    LinearArgs qkv{};
    qkv.x = fuse_in ? a.x : a.xn;
    if (fuse_in) {
      qkv.ssq_in = a.ssq;
      qkv.norm_g = w.ln1;
      qkv.norm_eps = kEps;
    }
    qkv.lda = d;
    qkv.w = w.wqkv;
    qkv.bias = w.bqkv;
    qkv.M = B;
    qkv.N = 3 * d;
    qkv.K = d;
    qkv.epi = EPI_QKV;
    qkv.qkv = QKVDst{a.q, kl, vl, pos, sb, sh, 1, m->H, m->dk, d};
    NML_TRY(launch_linear(m->dt, qkv, st));
    if (rope_on(m))
      NML_TRY(launch_rope(m->dt, a.q, kl, sb, sh, B, m->H, 1, m->dk, pos, nullptr, m->rope_cos,
                          m->rope_sin, m->P, st));
    AttnArgs at{};
    at.q = a.q;
    at.k = kl;
    at.v = vl;
    at.out = a.att;
    at.pos_base = pos;
    at.kv_stride_b = sb;
    at.kv_stride_h = sh;
    at.B = B;
    at.H = m->H;
    at.S = 1;
    at.dk = m->dk;
    at.scale = sqrtf((float)m->dk);
    NML_TRY(launch_attention_decode(m->dt, at, pos, max_len, a.part, st));
    LinearArgs wo{};
    wo.x = a.att;
    wo.lda = d;
    wo.w = w.wo;
    wo.bias = w.bo;
    wo.resid = a.x;
    wo.out = a.x;
    wo.M = B;
    wo.N = d;
    wo.K = d;
    wo.epi = EPI_BIAS_RESID;
    if (fuse) wo.ssq_out = a.ssq;
    NML_TRY(launch_linear(m->dt, wo, st));
    if (!fuse) NML_TRY(launch_rmsnorm(m->dt, a.x, w.ln2, a.xn, nullptr, nullptr, B, d, kEps, st));
    LinearArgs f1{};
    f1.x = fuse ? a.x : a.xn;
    if (fuse) {
      f1.ssq_in = a.ssq;
      f1.norm_g = w.ln2;
      f1.norm_eps = kEps;
    }
    f1.lda = d;
    f1.w = w.w1;
    f1.bias = w.b1;
    f1.out = a.h;
    f1.M = B;
    f1.N = m->F;
    f1.K = d;
    f1.epi = EPI_BIAS_GELU;
    NML_TRY(launch_linear(m->dt, f1, st));
    LinearArgs f2{};
    f2.x = a.h;
    f2.lda = m->F;
    f2.w = w.w2;
    f2.bias = w.b2;
    f2.resid = a.x;
    f2.out = a.x;
    f2.M = B;
    f2.N = d;
    f2.K = m->F;
    f2.epi = EPI_BIAS_RESID;
    if (fuse) f2.ssq_out = a.ssq;
    NML_TRY(launch_linear(m->dt, f2, st));
  }
  if (!fuse) NML_TRY(launch_rmsnorm(m->dt, a.x, m->lnf, a.xn, nullptr, nullptr, B, d, kEps, st));
  LinearArgs lm{};
  lm.x = fuse ? a.x : a.xn;
  if (fuse) {
    lm.ssq_in = a.ssq;
    lm.norm_g = m->lnf;
    lm.norm_eps = kEps;
  }
  lm.lda = d;
  lm.w = m->emb;
  lm.out = logits;
  lm.M = B;
  lm.N = m->V;
  lm.K = d;
  lm.epi = EPI_NONE;
  return launch_linear(m->dt, lm, st);
}

__global__ void set_u32_kernel(uint32_t* p, uint32_t v) {
  if (threadIdx.x == 0 && blockIdx.x == 0) p[0] = v;
}

// NIMBLEML_PERSISTENT=0 selects the multi-kernel decode step even where the
// persistent one applies.
bool persist_wanted() {
  const char* e = std::getenv("NIMBLEML_PERSISTENT");
  return !(e && e[0] == '0');
}

// Layer-0 parameter pointers with the per-layer stride, zeroed exchange slots and
// epoch = 1 for a persistent decode. Fails (so the caller uses the multi-kernel
// step) if the arena does not place every layer at one fixed stride.
int persist_prepare(nml_model* m, PersistArgs* pa, hipStream_t st) {
  const Layer& l0 = m->layers[0];
  const long long stride =
      m->L > 1 ? static_cast<const char*>(m->layers[1].ln1) - static_cast<const char*>(l0.ln1) : 0;
  for (int l = 1; l < m->L; ++l) {
    const Layer& w = m->layers[l];
    const void* const have[] = {w.ln1, w.wqkv, w.bqkv, w.wo, w.bo, w.ln2, w.w1, w.b1, w.w2, w.b2};
    const void* const first[] = {l0.ln1, l0.wqkv, l0.bqkv, l0.wo, l0.bo, l0.ln2, l0.w1, l0.b1, l0.w2, l0.b2};
    for (int k = 0; k < 10; ++k)
      NML_REQUIRE(static_cast<const char*>(have[k]) == static_cast<const char*>(first[k]) + l * stride,
                  "persistent decode: layer parameters are not at a fixed stride");
  }
  pa->ln1 = l0.ln1;
  pa->wqkv = l0.wqkv;
  pa->bqkv = l0.bqkv;
  pa->wo = l0.wo;
  pa->bo = l0.bo;
  pa->ln2 = l0.ln2;
  pa->w1 = l0.w1;
  pa->b1 = l0.b1;
  pa->w2 = l0.w2;
  pa->b2 = l0.b2;
  pa->layer_bytes = stride;
  const size_t sb = align256(persist_slot_count(m->d, m->H) * 8);
  NML_TRY(m->persist.ensure(sb + 256));
  char* base = static_cast<char*>(m->persist.p);
  NML_HIP(hipMemsetAsync(base, 0, sb + 256, st));
  uint32_t* epoch = reinterpret_cast<uint32_t*>(base + sb);
  set_u32_kernel<<<1, 64, 0, st>>>(epoch, 1u);
  NML_LAUNCHED();
  pa->slots = reinterpret_cast<unsigned long long*>(base);
  pa->epoch = epoch;
  return 0;
}

// Arguments of a persistent decode step over cache c (batch 1): feeds tokens[pos[0]]
// at position pos[0], writes the logits; fuse_argmax also writes the greedy choice to
// tokens[pos[0] + 1] and advances pos[0].
int persist_args(nml_model* m, nml_cache* c, int64_t* tokens, int32_t* pos, void* logits, int* err,
                 int fuse_argmax, PersistArgs* pa, hipStream_t st) {
  NML_TRY(persist_prepare(m, pa, st));
  pa->emb = m->emb;
  pa->posw = m->pos;
  pa->lnf = m->lnf;
  pa->kc = c->k;
  pa->vc = c->v;
  pa->kv_layer = (long long)c->B * m->H * m->P * m->dk;
  pa->kv_head = (long long)m->P * m->dk;
  pa->tokens = tokens;
  pa->pos = pos;
  pa->logits = logits;
  pa->err = err;
  pa->V = m->V;
  pa->L = m->L;
  pa->P = m->P;
  pa->fuse_argmax = fuse_argmax;
  pa->scale = sqrtf((float)m->dk);
  return 0;
}

__global__ void add_scalar_kernel(int32_t* p, int n, int v) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] += v;
}

// dst row b = src row row_start[b] + seq_len[b] − 1 (the last position of each packed
// sequence), rows of `bytes` bytes, a multiple of 16.
__global__ void gather_last_rows_kernel(const char* __restrict__ src, const int32_t* __restrict__ row_start,
                                        const int32_t* __restrict__ seq_len, char* __restrict__ dst,
                                        int bytes) {
  typedef int iv4 __attribute__((ext_vector_type(4)));
  const int b = blockIdx.x;
  const size_t r = static_cast<size_t>(row_start[b]) + seq_len[b] - 1;
  const iv4* s = reinterpret_cast<const iv4*>(src + r * bytes);
  iv4* o = reinterpret_cast<iv4*>(dst + static_cast<size_t>(b) * bytes);
  for (int i = threadIdx.x; i < bytes / 16; i += blockDim.x) o[i] = s[i];
}

// tok[b·P + pos[b]] = ids[b]: one fed token per row at the row's own position.
__global__ void scatter_step_tokens_kernel(const int64_t* __restrict__ ids, const int32_t* __restrict__ pos,
                                           int64_t* __restrict__ tok, int B, int P) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b < B) tok[static_cast<long long>(b) * P + pos[b]] = ids[b];
}

__global__ void copy_rows_kernel(const int64_t* __restrict__ src, long long sstride,
                                 int64_t* __restrict__ dst, long long dstride,
                                 const int32_t* __restrict__ lens) {
  const int b = blockIdx.x;
  const int n = lens[b];
  for (int i = threadIdx.x; i < n; i += blockDim.x) dst[b * dstride + i] = src[b * sstride + i];
}

// The fed-token buffer (B × P int64) and error word of single-token steps on cache c.
int cache_step_buffers(nml_model* m, nml_cache* c) {
  if (c->tok) return 0;
  void* p = nullptr;
  const size_t tb = align256((size_t)c->B * m->P * 8);
  NML_HIP(hipMalloc(&p, tb + 256));
  c->tok = static_cast<int64_t*>(p);
  c->err = reinterpret_cast<int*>(static_cast<char*>(p) + tb);
  return 0;
}

// Prefill of B prompts (device int64 rows at prompt_stride, host lengths plen) into
// cache c from position 0: one batched pass, prompts of different lengths packed row
// after row (the GEMMs see Σ plen rows, attention runs per sequence over its own length).
// Leaves each row's last-position logits (B, V) in `logits`; out-of-range ids set sm.err.
int prefill_rows(nml_model* m, nml_cache* c, const int64_t* prompts, size_t prompt_stride,
                 const std::vector<int32_t>& plen, const Small& sm, void* logits, hipStream_t st) {
  const int B = (int)plen.size();
  int maxp = 0;
  bool same = true;
  for (int b = 0; b < B; ++b) {
    maxp = plen[b] > maxp ? plen[b] : maxp;
    same = same && plen[b] == plen[0];
  }
  const size_t layer_kv = (size_t)B * m->H * m->P * m->dk * m->es;
  const long long sb = (long long)m->H * m->P * m->dk, sh = (long long)m->P * m->dk;
  NML_HIP(hipMemsetAsync(sm.zeros, 0, B * 4, st));
  if (same) {
    const int S = plen[0];
    Acts a;
    NML_TRY(acts_for(m, B * S, B, &a));
    if ((int)prompt_stride != S) {
      for (int b = 0; b < B; ++b)
        NML_TRY(launch_embed(m->dt, prompts + (size_t)b * prompt_stride, m->emb, posw(m), nullptr,
                             static_cast<char*>(a.x) + (size_t)b * S * m->d * m->es, 1, S, m->d,
                             m->V, m->P, sm.err, st));
    } else {
      NML_TRY(launch_embed(m->dt, prompts, m->emb, posw(m), nullptr, a.x, B, S, m->d, m->V, m->P,
                           sm.err, st));
    }
    NML_TRY(trunk(m, a, B, S, sm.zeros,
                  [&](int l) {
                    return KVView{static_cast<char*>(c->k) + l * layer_kv,
                                  static_cast<char*>(c->v) + l * layer_kv, sb, sh};
                  },
                  st));
    NML_TRY(head(m, a, B, S, logits, 1, st));
  } else {
    // Packed rows: (b << 16) | s per row, then the lengths and row starts.
    std::vector<int32_t> tab;
    int R = 0;
    for (int b = 0; b < B; ++b) R += plen[b];
    NML_REQUIRE(maxp < 65536 && B < 32768, "ragged prefill: %d prompts up to %d long", B, maxp);
    NML_REQUIRE(((size_t)m->d * m->es) % 16 == 0, "ragged prefill: row of %d not 16-byte sized", m->d);
    tab.reserve((size_t)R + 2 * B + 1);
    for (int b = 0; b < B; ++b)
      for (int s = 0; s < plen[b]; ++s) tab.push_back((b << 16) | s);
    tab.insert(tab.end(), plen.begin(), plen.end());
    std::vector<int32_t> starts(B);
    for (int b = 0, r = 0; b < B; r += plen[b], ++b) starts[b] = r;
    tab.insert(tab.end(), starts.begin(), starts.end());
    NML_TRY(m->ragged.ensure(tab.size() * 4));
    const int32_t* dtab = static_cast<const int32_t*>(m->ragged.p);
    NML_HIP(hipMemcpyAsync(m->ragged.p, tab.data(), tab.size() * 4, hipMemcpyHostToDevice, st));
    const Ragged rg{dtab, dtab + R, dtab + R + B, R};
    // activations sized for the padded (B, maxp) query layout
    Acts a;
    NML_TRY(acts_for(m, B * maxp, B, &a));
    for (int b = 0; b < B; ++b)
      NML_TRY(launch_embed(m->dt, prompts + (size_t)b * prompt_stride, m->emb, posw(m), nullptr,
                           static_cast<char*>(a.x) + (size_t)starts[b] * m->d * m->es, 1, plen[b],
                           m->d, m->V, m->P, sm.err, st));
    NML_TRY(trunk(m, a, B, maxp, sm.zeros,
                  [&](int l) {
                    return KVView{static_cast<char*>(c->k) + l * layer_kv,
                                  static_cast<char*>(c->v) + l * layer_kv, sb, sh};
                  },
                  st, &rg));
    gather_last_rows_kernel<<<B, 128, 0, st>>>(static_cast<const char*>(a.xn), rg.row_start,
                                               rg.seq_len, static_cast<char*>(a.att),
                                               m->d * (int)m->es);
    NML_LAUNCHED();
    Acts last = a;
    last.xn = a.att;
    NML_TRY(head(m, last, B, 1, logits, 1, st));
  }
  return 0;
}

// One token per row (device int64 ids, (B)) at each row's own position c->len[b],
// through generate()'s decode step (decode_step: the skinny projections with the fused
// norms, split-K attention over the cache, the tied head); logits (B, V). Advances every
// row by one position; reports an out-of-range id.
int decode_rows(nml_model* m, nml_cache* c, const int64_t* ids, void* logits, hipStream_t st) {
  const int B = c->B;
  int maxlen = 0;
  for (int v : c->len) maxlen = v > maxlen ? v : maxlen;
  NML_REQUIRE(maxlen + 1 <= m->P, "Sequence length %d exceeds maximum sequence length %d",
              maxlen + 1, m->P);
  NML_TRY(cache_step_buffers(m, c));
  scatter_step_tokens_kernel<<<(B + 255) / 256, 256, 0, st>>>(ids, c->len_dev, c->tok, B, m->P);
  NML_LAUNCHED();
  NML_HIP(hipMemsetAsync(c->err, 0, sizeof(int), st));
  Acts a;
  NML_TRY(acts_for(m, B, B, &a));
  // the workspace is shared with other forwards: clear the attention partials each call
  NML_HIP(hipMemsetAsync(a.part, 0, attention_decode_workspace(B, m->H, m->dk, m->P), st));
  NML_TRY(decode_step(m, c, a, 0, B, c->tok, m->P, c->len_dev, c->err, logits, maxlen + 1, st));
  add_scalar_kernel<<<(B + 255) / 256, 256, 0, st>>>(c->len_dev, B, 1);
  NML_LAUNCHED();
  for (auto& v : c->len) v += 1;
  int herr = 0;
  NML_HIP(hipMemcpyAsync(&herr, c->err, sizeof(int), hipMemcpyDeviceToHost, st));
  NML_HIP(hipStreamSynchronize(st));
  m->last_decode_persistent = 0;
  NML_REQUIRE(herr == 0, "Token ID out of range [0, %d)", m->V);
  return 0;
}

}  // namespace

extern "C" {

int nml_model_create(int vocab, int d_model, int num_heads, int num_layers, int max_seq_len,
                     int d_ff, int dtype, nml_model** out) {
  *out = nullptr;
  NML_REQUIRE(dtype == F32 || dtype == F16, "dtype must be 0 or 1");
  NML_REQUIRE(vocab > 0 && d_model > 0 && num_heads > 0 && num_layers > 0 && max_seq_len > 0 &&
                  d_ff > 0,
              "model dimensions must be positive");
  NML_REQUIRE(d_model % num_heads == 0, "d_model (%d) must be divisible by num_heads (%d).",
              d_model, num_heads);
  NML_REQUIRE(d_model / num_heads <= kMaxHeadDim, "head_dim %d above %d (d_model / num_heads)",
              d_model / num_heads, kMaxHeadDim);
  const int vec = dtype == F16 ? 8 : 4;
  NML_REQUIRE(d_model % vec == 0 && d_ff % vec == 0,
              "d_model and d_ff must be multiples of %d for 16-byte loads", vec);
  nml_model* m = new nml_model();
  m->V = vocab;
  m->d = d_model;
  m->H = num_heads;
  m->L = num_layers;
  m->P = max_seq_len;
  m->F = d_ff;
  m->dt = dtype;
  m->dk = d_model / num_heads;
  m->es = dtype_size(dtype);
  m->layers.resize(num_layers);
  size_t total = align256(param_elems(m, NML_P_TOKEN_EMB) * m->es) +
                 align256(param_elems(m, NML_P_POS_EMB) * m->es) +
                 align256(param_elems(m, NML_P_LN_F) * m->es) +
                 2 * align256(param_elems(m, NML_P_ROPE_COS) * m->es);
  for (int k : kLayerKinds) total += (size_t)num_layers * align256(param_elems(m, k) * m->es);
  hipError_t e = hipMalloc(&m->arena, total);
  if (e != hipSuccess) {
    set_error("model: hipMalloc(%zu) failed: %s", total, hipGetErrorString(e));
    delete m;
    return -1;
  }
  m->arena_bytes = total;
  // Split-K workspace of the batched-decode projections (before any graph capture).
  if (linear_reserve_workspace(4096) != 0) {
    (void)hipFree(m->arena);
    delete m;
    return -1;
  }
  char* p = static_cast<char*>(m->arena);
  auto take = [&](int kind, int layer) {
    void** slot = param_slot(m, kind, layer);
    *slot = p;
    p += align256(param_elems(m, kind) * m->es);
  };
  take(NML_P_TOKEN_EMB, 0);
  take(NML_P_POS_EMB, 0);
  take(NML_P_LN_F, 0);
  take(NML_P_ROPE_COS, 0);
  take(NML_P_ROPE_SIN, 0);
  for (int l = 0; l < num_layers; ++l)
    for (int k : kLayerKinds) take(k, l);
  *out = m;
  return 0;
}

int nml_model_destroy(nml_model* m) {
  if (!m) return 0;
  (void)hipStreamSynchronize(nml::stream());
  m->ws.release();
  m->ws2.release();
  m->kvs.release();
  m->logits_ws.release();
  m->small.release();
  m->persist.release();
  m->ragged.release();
  train_release(m);
  if (m->arena) (void)hipFree(m->arena);
  delete m;
  return 0;
}

int nml_model_set_param(nml_model* m, int kind, int layer, const void* host, size_t bytes) {
  NML_REQUIRE(m != nullptr, "model is null");
  void** slot = param_slot(m, kind, layer);
  NML_REQUIRE(slot != nullptr, "unknown parameter kind %d / layer %d", kind, layer);
  const size_t want = param_elems(m, kind) * m->es;
  NML_REQUIRE(bytes == want, "parameter kind %d: expected %zu bytes, got %zu", kind, want, bytes);
  NML_HIP(hipMemcpyAsync(*slot, host, bytes, hipMemcpyHostToDevice, nml::stream()));
  NML_TRY(train_param_uploaded(m, *slot, param_elems(m, kind)));
  NML_HIP(hipStreamSynchronize(nml::stream()));
  if (kind == NML_P_ROPE_COS) m->rope_cos_set = true;
  if (kind == NML_P_ROPE_SIN) m->rope_sin_set = true;
  return 0;
}

int nml_model_param_ptr(nml_model* m, int kind, int layer, void** ptr) {
  NML_REQUIRE(m != nullptr, "model is null");
  void** slot = param_slot(m, kind, layer);
  NML_REQUIRE(slot != nullptr, "unknown parameter kind %d / layer %d", kind, layer);
  *ptr = *slot;
  return 0;
}

int nml_model_forward(nml_model* m, const int64_t* ids, size_t batch, size_t seq, void* logits,
                      int last_only) {
  NML_TRY(check_ready(m));
  NML_REQUIRE(seq <= (size_t)m->P, "Sequence length %zu exceeds maximum sequence length %d", seq,
              m->P);
  if (batch == 0 || seq == 0) return 0;
  const int B = (int)batch, S = (int)seq;
  hipStream_t st = nml::stream();
  Acts a;
  NML_TRY(acts_for(m, B * S, 0, &a));
  const size_t kvb = align256((size_t)B * S * m->d * m->es);
  NML_TRY(m->kvs.ensure(2 * kvb));
  void* kbuf = m->kvs.p;
  void* vbuf = static_cast<char*>(m->kvs.p) + kvb;
  NML_TRY(launch_embed(m->dt, ids, m->emb, posw(m), nullptr, a.x, B, S, m->d, m->V, m->P, nullptr,
                       st));
  const long long sb = (long long)m->H * S * m->dk, sh = (long long)S * m->dk;
  NML_TRY(trunk(m, a, B, S, nullptr, [&](int) { return KVView{kbuf, vbuf, sb, sh}; }, st));
  return head(m, a, B, S, logits, last_only, st);
}

int nml_model_blocks_forward(nml_model* m, const void* x, void* out, size_t batch, size_t seq,
                             int final_norm, int causal, const void* mask) {
  NML_REQUIRE(m != nullptr, "model is null");
  NML_REQUIRE(seq <= (size_t)m->P, "Sequence length %zu exceeds maximum sequence length %d", seq,
              m->P);
  NML_REQUIRE(!causal || mask == nullptr, "blocks_forward: a causal call takes no mask");
  if (batch == 0 || seq == 0) return 0;
  const int B = (int)batch, S = (int)seq;
  hipStream_t st = nml::stream();
  Acts a;
  NML_TRY(acts_for(m, B * S, 0, &a));
  const size_t bytes = (size_t)B * S * m->d * m->es;
  const size_t kvb = align256(bytes);
  NML_TRY(m->kvs.ensure(2 * kvb));
  void* kbuf = m->kvs.p;
  void* vbuf = static_cast<char*>(m->kvs.p) + kvb;
  NML_HIP(hipMemcpyAsync(a.x, x, bytes, hipMemcpyDeviceToDevice, st));
  AttnMode am;
  am.full = causal ? 0 : 1;
  am.mask = mask;
  const long long sb = (long long)m->H * S * m->dk, sh = (long long)S * m->dk;
  NML_TRY(trunk(m, a, B, S, nullptr, [&](int) { return KVView{kbuf, vbuf, sb, sh}; }, st,
                nullptr, final_norm != 0, am));
  NML_HIP(hipMemcpyAsync(out, final_norm ? a.xn : a.x, bytes, hipMemcpyDeviceToDevice, st));
  return 0;
}

int nml_model_mha_forward(nml_model* m, int layer, const void* x, void* out, size_t batch,
                          size_t seq, int causal, const void* mask) {
  NML_REQUIRE(m != nullptr, "model is null");
  NML_REQUIRE(layer >= 0 && layer < m->L, "layer %d outside [0, %d)", layer, m->L);
  NML_REQUIRE(seq <= (size_t)m->P, "Sequence length %zu exceeds maximum sequence length %d", seq,
              m->P);
  NML_REQUIRE(!causal || mask == nullptr, "mha_forward: a causal call takes no mask");
  if (batch == 0 || seq == 0) return 0;
  const int B = (int)batch, S = (int)seq;
  hipStream_t st = nml::stream();
  Acts a;
  NML_TRY(acts_for(m, B * S, 0, &a));
  const size_t kvb = align256((size_t)B * S * m->d * m->es);
  NML_TRY(m->kvs.ensure(2 * kvb));
  AttnMode am;
  am.full = causal ? 0 : 1;
  am.mask = mask;
  const long long sb = (long long)m->H * S * m->dk, sh = (long long)S * m->dk;
  const KVView c{m->kvs.p, static_cast<char*>(m->kvs.p) + kvb, sb, sh};
  // neural_network/attention.py:139-168 applies no rotary embedding
  return attention_sublayer(m, m->layers[layer], x, a, B, S, nullptr, c, false, am, nullptr, out,
                            st, nullptr);
}

// Mean of the accumulated row losses → *loss, with the embedding and label range checks.
static int finish_loss(nml_model* m, const Small& sm, hipStream_t st, double* loss) {
  NML_TRY(launch_ce_finalize(sm.acc, sm.acc + 2, st));
  double host[3];
  int herr = 0;
  NML_HIP(hipMemcpyAsync(host, sm.acc, sizeof(host), hipMemcpyDeviceToHost, st));
  NML_HIP(hipMemcpyAsync(&herr, sm.err, sizeof(int), hipMemcpyDeviceToHost, st));
  NML_HIP(hipStreamSynchronize(st));
  NML_REQUIRE((herr & 1) == 0, "Token ID out of range [0, %d)", m->V);
  NML_REQUIRE((herr & 2) == 0, "label out of range [0, %d)", m->V);
  *loss = host[2];
  return 0;
}

int nml_model_loss(nml_model* m, const int64_t* ids, const int64_t* labels, size_t batch,
                   size_t seq, int64_t ignore_index, int has_ignore, double* loss) {
  NML_TRY(check_ready(m));
  NML_REQUIRE(seq <= (size_t)m->P, "Sequence length %zu exceeds maximum sequence length %d", seq,
              m->P);
  const int B = (int)batch, S = (int)seq, R = B * S;
  if (R == 0) {
    *loss = 0.0;
    return 0;
  }
  hipStream_t st = nml::stream();
  Acts a;
  NML_TRY(acts_for(m, R, 0, &a));
  const size_t kvb = align256((size_t)R * m->d * m->es);
  NML_TRY(m->kvs.ensure(2 * kvb));
  void* kbuf = m->kvs.p;
  void* vbuf = static_cast<char*>(m->kvs.p) + kvb;
  Small sm;
  NML_TRY(small_for(m, 1, &sm));
  NML_HIP(hipMemsetAsync(sm.err, 0, sizeof(int), st));
  NML_TRY(launch_embed(m->dt, ids, m->emb, posw(m), nullptr, a.x, B, S, m->d, m->V, m->P, sm.err,
                       st));
  const long long sb = (long long)m->H * S * m->dk, sh = (long long)S * m->dk;
  NML_TRY(trunk(m, a, B, S, nullptr, [&](int) { return KVView{kbuf, vbuf, sb, sh}; }, st));
  if (linear_ce_fusable(m->dt, R, m->d, m->V)) {
    // fp16 at prefill sizes: the head GEMM's epilogue forms each row's softmax partials
    // per 256-column tile and the label's logit; no logits are stored.
    const int tn = (m->V + kLinearCETile - 1) / kLinearCETile;
    const size_t pb = align256((size_t)R * tn * sizeof(float2));
    const size_t rb = align256((size_t)R * 4);
    NML_TRY(m->logits_ws.ensure(pb + 3 * rb));
    char* w = static_cast<char*>(m->logits_ws.p);
    float2* part = reinterpret_cast<float2*>(w);
    float* label_logit = reinterpret_cast<float*>(w + pb);
    float* row_loss = reinterpret_cast<float*>(w + pb + rb);
    int* row_valid = reinterpret_cast<int*>(w + pb + 2 * rb);
    LinearArgs lm{};
    lm.x = a.xn;
    lm.lda = m->d;
    lm.w = m->emb;
    lm.M = R;
    lm.N = m->V;
    lm.K = m->d;
    lm.epi = EPI_CE;
    lm.ce = CEDst{labels, part, label_logit, tn};
    NML_TRY(launch_linear(m->dt, lm, st));
    NML_TRY(launch_ce_combine(part, tn, label_logit, R, m->V, labels, ignore_index, has_ignore,
                              row_loss, row_valid, sm.err, st));
    NML_TRY(launch_ce_reduce(row_loss, row_valid, R, sm.acc, 0, st));
    return finish_loss(m, sm, st, loss);
  }
  // Logits in row chunks of ≤ 512 MiB, never all (R, V) at once.
  size_t chunk = R;
  while (chunk > 1 && chunk * m->V * m->es > ((size_t)512 << 20)) chunk = (chunk + 1) / 2;
  const size_t lb = align256(chunk * m->V * m->es);
  const size_t rb = align256((size_t)R * 4);
  NML_TRY(m->logits_ws.ensure(lb + 2 * rb));
  void* lg = m->logits_ws.p;
  float* row_loss = reinterpret_cast<float*>(static_cast<char*>(m->logits_ws.p) + lb);
  int* row_valid = reinterpret_cast<int*>(static_cast<char*>(m->logits_ws.p) + lb + rb);
  for (size_t r0 = 0; r0 < (size_t)R; r0 += chunk) {
    const int n = (int)(((size_t)R - r0 < chunk) ? (size_t)R - r0 : chunk);
    LinearArgs lm{};
    lm.x = static_cast<const char*>(a.xn) + r0 * m->d * m->es;
    lm.lda = m->d;
    lm.w = m->emb;
    lm.out = lg;
    lm.M = n;
    lm.N = m->V;
    lm.K = m->d;
    lm.epi = EPI_NONE;
    NML_TRY(launch_linear(m->dt, lm, st));
    NML_TRY(launch_ce_rows(m->dt, lg, n, m->V, labels + r0, ignore_index, has_ignore, row_loss,
                           row_valid, sm.err, st));
    NML_TRY(launch_ce_reduce(row_loss, row_valid, n, sm.acc, r0 > 0, st));
  }
  return finish_loss(m, sm, st, loss);
}

int nml_cache_create(nml_model* m, size_t batch, nml_cache** out) {
  *out = nullptr;
  NML_TRY(check_ready(m));
  NML_REQUIRE(batch > 0 && batch <= 4096, "cache batch %zu out of range", batch);
  nml_cache* c = new nml_cache();
  c->m = m;
  c->B = (int)batch;
  const size_t bytes = (size_t)m->L * batch * m->H * m->P * m->dk * m->es;
  hipError_t e1 = hipMalloc(&c->k, bytes);
  hipError_t e2 = e1 == hipSuccess ? hipMalloc(&c->v, bytes) : e1;
  hipError_t e3 = e2 == hipSuccess ? hipMalloc(&c->len_dev, align256(batch * 4)) : e2;
  if (e3 != hipSuccess) {
    set_error("cache: allocation of 2 × %zu bytes failed: %s", bytes, hipGetErrorString(e3));
    if (c->k) (void)hipFree(c->k);
    if (c->v) (void)hipFree(c->v);
    delete c;
    return -1;
  }
  c->len.assign(batch, 0);
  NML_HIP(hipMemsetAsync(c->len_dev, 0, batch * 4, nml::stream()));
  *out = c;
  return 0;
}

int nml_cache_destroy(nml_cache* c) {
  if (!c) return 0;
  (void)hipStreamSynchronize(nml::stream());
  if (c->k) (void)hipFree(c->k);
  if (c->v) (void)hipFree(c->v);
  if (c->len_dev) (void)hipFree(c->len_dev);
  if (c->tok) (void)hipFree(c->tok);
  delete c;
  return 0;
}

int nml_cache_length(nml_cache* c, size_t* len) {
  NML_REQUIRE(c != nullptr, "cache is null");
  *len = c->len.empty() ? 0 : (size_t)c->len[0];
  return 0;
}

int nml_model_forward_cached(nml_model* m, nml_cache* c, const int64_t* ids, size_t batch,
                             size_t seq, void* logits, int last_only) {
  NML_TRY(check_ready(m));
  NML_REQUIRE(c != nullptr && c->m == m, "cache does not belong to this model");
  NML_REQUIRE((int)batch == c->B, "batch %zu does not match the cache batch %d", batch, c->B);
  const int B = (int)batch, S = (int)seq;
  if (S == 0) return 0;
  int start = 0;  // the longest row (rows prefilled ragged sit at different positions)
  for (int v : c->len) start = v > start ? v : start;
  NML_REQUIRE((size_t)start + seq <= (size_t)m->P,
              "Sequence length %zu exceeds maximum sequence length %d", start + seq, m->P);
  hipStream_t st = nml::stream();
  if (B == 1 && S == 1 && persist_wanted() && !rope_on(m) &&
      persist_supported(m->dt, m->d, m->H, m->F, B, m->P)) {
    // One token of one sequence: the persistent decode kernel (logits out, no choice).
    NML_TRY(cache_step_buffers(m, c));
    NML_HIP(hipMemcpyAsync(c->tok + start, ids, sizeof(int64_t), hipMemcpyDeviceToDevice, st));
    NML_HIP(hipMemsetAsync(c->err, 0, sizeof(int), st));
    PersistArgs pa{};
    NML_TRY(persist_args(m, c, c->tok, c->len_dev, logits, c->err, 0, &pa, st));
    NML_TRY(launch_decode_persist(m->dt, m->d, m->H, pa, st));
    add_scalar_kernel<<<1, 64, 0, st>>>(c->len_dev, 1, 1);
    NML_LAUNCHED();
    c->len[0] += 1;
    int herr = 0;
    NML_HIP(hipMemcpyAsync(&herr, c->err, sizeof(int), hipMemcpyDeviceToHost, st));
    NML_HIP(hipStreamSynchronize(st));
    m->last_decode_persistent = 1;
    NML_REQUIRE((herr & 4) == 0, "persistent decode: a data exchange timed out");
    NML_REQUIRE(herr == 0, "Token ID out of range [0, %d)", m->V);
    return 0;
  }
  // one token per row: generate()'s decode step (rows may sit at different positions)
  if (S == 1) return decode_rows(m, c, ids, logits, st);
  Acts a;
  NML_TRY(acts_for(m, B * S, 0, &a));
  NML_TRY(launch_embed(m->dt, ids, m->emb, posw(m), c->len_dev, a.x, B, S, m->d, m->V, m->P,
                       nullptr, st));
  const size_t layer_kv = (size_t)B * m->H * m->P * m->dk * m->es;
  const long long sb = (long long)m->H * m->P * m->dk, sh = (long long)m->P * m->dk;
  NML_TRY(trunk(m, a, B, S, c->len_dev,
                [&](int l) {
                  return KVView{static_cast<char*>(c->k) + l * layer_kv,
                                static_cast<char*>(c->v) + l * layer_kv, sb, sh};
                },
                st));
  NML_TRY(head(m, a, B, S, logits, last_only, st));
  add_scalar_kernel<<<(B + 255) / 256, 256, 0, st>>>(c->len_dev, B, S);
  NML_LAUNCHED();
  for (auto& v : c->len) v += S;
  return 0;
}

int nml_model_prefill_ragged(nml_model* m, nml_cache* c, const int64_t* prompts,
                             size_t prompt_stride, const int32_t* prompt_len, size_t batch,
                             void* logits) {
  NML_TRY(check_ready(m));
  NML_REQUIRE(c != nullptr && c->m == m, "cache does not belong to this model");
  NML_REQUIRE((int)batch == c->B, "batch %zu does not match the cache batch %d", batch, c->B);
  for (int v : c->len) NML_REQUIRE(v == 0, "prefill_ragged: the cache is not empty");
  const int B = (int)batch;
  std::vector<int32_t> plen(prompt_len, prompt_len + B);
  for (int b = 0; b < B; ++b) {
    NML_REQUIRE(plen[b] > 0, "prompt %d is empty", b);
    NML_REQUIRE((size_t)plen[b] <= prompt_stride, "prompt %d longer than its stride", b);
    NML_REQUIRE(plen[b] <= m->P, "Sequence length %d exceeds maximum sequence length %d", plen[b],
                m->P);
  }
  hipStream_t st = nml::stream();
  Small sm;
  NML_TRY(small_for(m, B, &sm));
  NML_HIP(hipMemsetAsync(sm.err, 0, sizeof(int), st));
  NML_TRY(prefill_rows(m, c, prompts, prompt_stride, plen, sm, logits, st));
  NML_HIP(hipMemcpyAsync(c->len_dev, plen.data(), B * 4, hipMemcpyHostToDevice, st));
  int herr = 0;
  NML_HIP(hipMemcpyAsync(&herr, sm.err, sizeof(int), hipMemcpyDeviceToHost, st));
  NML_HIP(hipStreamSynchronize(st));  // plen (host) is read by the copy above
  c->len = plen;
  NML_REQUIRE(herr == 0, "Token ID out of range [0, %d)", m->V);
  return 0;
}

int nml_model_generate(nml_model* m, const int64_t* prompts, size_t prompt_stride,
                       const int32_t* prompt_len, size_t batch, size_t max_new,
                       float temperature, int top_k, float top_p, float repetition_penalty,
                       const double* u, int64_t* tokens_out, size_t out_stride, int use_graph) {
  NML_TRY(check_ready(m));
  const int B = (int)batch;
  if (B == 0 || max_new == 0) return 0;
  int maxp = 0;
  bool same = true;
  for (int b = 0; b < B; ++b) {
    NML_REQUIRE(prompt_len[b] > 0, "prompt %d is empty", b);
    NML_REQUIRE((size_t)prompt_len[b] <= prompt_stride, "prompt %d longer than its stride", b);
    maxp = prompt_len[b] > maxp ? prompt_len[b] : maxp;
    same = same && prompt_len[b] == prompt_len[0];
    // The reference re-forwards the whole sequence before each new token; its last
    // forward covers prompt_len + max_new − 1 tokens (models/gpt.py:82-83).
    NML_REQUIRE((size_t)prompt_len[b] + max_new - 1 <= (size_t)m->P,
                "Sequence length %zu exceeds maximum sequence length %d",
                (size_t)prompt_len[b] + max_new - 1, m->P);
  }
  NML_REQUIRE(out_stride >= (size_t)maxp + max_new, "tokens_out stride too small");
  NML_REQUIRE(temperature <= 0.f || u != nullptr, "uniforms required for sampling");
  hipStream_t st = nml::stream();

  nml_cache* c = nullptr;
  NML_TRY(nml_cache_create(m, batch, &c));
  struct Guard {
    nml_cache* c;
    ~Guard() { nml_cache_destroy(c); }
  } guard{c};

  Small sm;
  NML_TRY(small_for(m, B, &sm));
  std::vector<int32_t> plen(prompt_len, prompt_len + B);
  NML_HIP(hipMemcpyAsync(sm.plen, plen.data(), B * 4, hipMemcpyHostToDevice, st));
  NML_HIP(hipMemsetAsync(sm.err, 0, sizeof(int), st));
  copy_rows_kernel<<<B, 256, 0, st>>>(prompts, (long long)prompt_stride, tokens_out,
                                      (long long)out_stride, sm.plen);
  NML_LAUNCHED();

  // Logits for the batch (B, V).
  const size_t lb = align256((size_t)B * m->V * m->es);
  NML_TRY(m->logits_ws.ensure(lb));
  void* logits = m->logits_ws.p;

  NML_TRY(prefill_rows(m, c, prompts, prompt_stride, plen, sm, logits, st));
  // pos[b] = prompt_len[b] − 1, then the first choice advances it to prompt_len[b].
  std::vector<int32_t> pos0(B);
  for (int b = 0; b < B; ++b) pos0[b] = plen[b] - 1;
  NML_HIP(hipMemcpyAsync(sm.pos, pos0.data(), B * 4, hipMemcpyHostToDevice, st));

  SampleArgs sa{};
  sa.logits = logits;
  sa.logits_stride = m->V;
  sa.B = B;
  sa.V = m->V;
  sa.temperature = temperature;
  sa.top_k = top_k;
  sa.top_p = top_p;
  sa.rep_penalty = repetition_penalty;
  sa.uniforms = u;
  sa.tokens = tokens_out;
  sa.tok_stride = (long long)out_stride;
  sa.pos = sm.pos;
  sa.plen = sm.plen;
  NML_TRY(launch_sample(m->dt, sa, st));

  // Batched decode in two halves on two streams (NIMBLEML_DECODE_SPLIT=0: one): one
  // half's latency-bound projections run beside the other half's bandwidth-bound
  // attention. Each half has its own activations and attention workspace.
  const char* se = std::getenv("NIMBLEML_DECODE_SPLIT");
  const bool split = !(se && se[0] == '0') && B >= 16 && B % 2 == 0;
  const int BA = split ? B / 2 : B;
  Acts a, a2;
  NML_TRY(acts_for(m, BA, BA, &a));
  NML_HIP(hipMemsetAsync(a.part, 0, attention_decode_workspace(BA, m->H, m->dk, m->P), st));
  hipStream_t st2 = nullptr;
  hipEvent_t ev_fork = nullptr, ev_join = nullptr;
  struct EvGuard {
    hipEvent_t* e[2];
    ~EvGuard() {
      for (hipEvent_t* p : e)
        if (*p) (void)hipEventDestroy(*p);
    }
  } ev_guard{{&ev_fork, &ev_join}};
  if (split) {
    NML_TRY(acts_in(m, m->ws2, BA, BA, &a2));
    NML_HIP(hipMemsetAsync(a2.part, 0, attention_decode_workspace(BA, m->H, m->dk, m->P), st));
    st2 = nml::stream2();
    NML_REQUIRE(st2 != nullptr, "decode: second stream unavailable");
    NML_HIP(hipEventCreateWithFlags(&ev_fork, hipEventDisableTiming));
    NML_HIP(hipEventCreateWithFlags(&ev_join, hipEventDisableTiming));
  }
  // Attention length bound of the decode steps: the last step feeds position
  // maxp + max_new - 2 and attends to every key up to it.
  const int decode_len = maxp + (int)max_new - 1;
  const bool persistent = persist_wanted() && !rope_on(m) &&
                          persist_supported(m->dt, m->d, m->H, m->F, B, m->P);
  PersistArgs pa{};
  if (persistent)
    NML_TRY(persist_args(m, c, tokens_out, sm.pos, logits, sm.err,
                         (temperature <= 0.f && repetition_penalty == 1.0f) ? 1 : 0, &pa, st));
  // NIMBLEML_PERSIST_TRACE=<file>: phase timestamps of the last persistent step.
  const char* trace_path = persistent ? std::getenv("NIMBLEML_PERSIST_TRACE") : nullptr;
  const size_t trace_n = (size_t)kPersistGroups * persist_trace_stride(m->L);
  Buf trace_buf;
  struct TraceGuard {
    Buf* b;
    ~TraceGuard() { b->release(); }
  } trace_guard{&trace_buf};
  if (trace_path && trace_path[0]) {
    NML_TRY(trace_buf.ensure(trace_n * 8));
    NML_HIP(hipMemsetAsync(trace_buf.p, 0, trace_n * 8, st));
    pa.trace = static_cast<unsigned long long*>(trace_buf.p);
  }
  // One decode step: feed tokens[pos], choose tokens[pos + 1], advance pos.
  auto step = [&]() -> int {
    if (persistent) {
      NML_TRY(launch_decode_persist(m->dt, m->d, m->H, pa, st));
      return pa.fuse_argmax ? 0 : launch_sample(m->dt, sa, st);
    }
    if (split) {  // fork: rows [BA, B) on the second stream, then join before sampling
      NML_HIP(hipEventRecord(ev_fork, st));
      NML_HIP(hipStreamWaitEvent(st2, ev_fork, 0));
      NML_TRY(decode_step(m, c, a2, BA, B - BA, tokens_out, (long long)out_stride, sm.pos, sm.err,
                          logits, decode_len, st2));
      NML_TRY(decode_step(m, c, a, 0, BA, tokens_out, (long long)out_stride, sm.pos, sm.err,
                          logits, decode_len, st));
      NML_HIP(hipEventRecord(ev_join, st2));
      NML_HIP(hipStreamWaitEvent(st, ev_join, 0));
      return launch_sample(m->dt, sa, st);
    }
    NML_TRY(decode_step(m, c, a, 0, B, tokens_out, (long long)out_stride, sm.pos, sm.err, logits,
                        decode_len, st));
    return launch_sample(m->dt, sa, st);
  };
  hipEvent_t e0 = nullptr, e1 = nullptr;
  NML_HIP(hipEventCreate(&e0));
  NML_HIP(hipEventCreate(&e1));
  const int steps = (int)max_new - 1;
  int rc = 0;
  if (steps > 0) {
    if (use_graph) {
      hipGraph_t graph = nullptr;
      hipGraphExec_t exec = nullptr;
      // G steps per graph (fewer launches; each step reads the position the previous one
      // advanced on the device), the remainder one step per launch of a second graph
      const char* ge = std::getenv("NIMBLEML_GRAPH_STEPS");
      const int G = std::max(1, std::min(steps, ge ? atoi(ge) : 8));
      hipGraph_t graph1 = nullptr;
      hipGraphExec_t exec1 = nullptr;
      int r1 = 0;
      NML_HIP(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
      for (int i = 0; i < G && r1 == 0; ++i) r1 = step();
      hipError_t ec = hipStreamEndCapture(st, &graph);
      if (r1 != 0) {
        if (graph) (void)hipGraphDestroy(graph);
        return -1;
      }
      NML_HIP(ec);
      NML_HIP(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0));
      if (steps % G) {
        NML_HIP(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
        r1 = step();
        ec = hipStreamEndCapture(st, &graph1);
        if (r1 != 0) {
          if (graph1) (void)hipGraphDestroy(graph1);
          (void)hipGraphExecDestroy(exec);
          (void)hipGraphDestroy(graph);
          return -1;
        }
        NML_HIP(ec);
        NML_HIP(hipGraphInstantiate(&exec1, graph1, nullptr, nullptr, 0));
      }
      NML_HIP(hipEventRecord(e0, st));
      for (int t = 0; t + G <= steps && rc == 0; t += G)
        if (hipGraphLaunch(exec, st) != hipSuccess) rc = -1;
      for (int t = 0; t < steps % G && rc == 0; ++t)
        if (hipGraphLaunch(exec1, st) != hipSuccess) rc = -1;
      NML_HIP(hipEventRecord(e1, st));
      (void)hipStreamSynchronize(st);
      (void)hipGraphExecDestroy(exec);
      (void)hipGraphDestroy(graph);
      if (exec1) (void)hipGraphExecDestroy(exec1);
      if (graph1) (void)hipGraphDestroy(graph1);
      NML_REQUIRE(rc == 0, "hipGraphLaunch failed");
    } else {
      NML_HIP(hipEventRecord(e0, st));
      for (int t = 0; t < steps; ++t) NML_TRY(step());
      NML_HIP(hipEventRecord(e1, st));
    }
  } else {
    NML_HIP(hipEventRecord(e0, st));
    NML_HIP(hipEventRecord(e1, st));
  }
  int herr = 0;
  NML_HIP(hipMemcpyAsync(&herr, sm.err, sizeof(int), hipMemcpyDeviceToHost, st));
  NML_HIP(hipStreamSynchronize(st));
  float ms = 0.f;
  NML_HIP(hipEventElapsedTime(&ms, e0, e1));
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  m->last_decode_ms = ms;
  m->last_decode_steps = steps;
  m->last_decode_persistent = persistent ? 1 : 0;
  if (pa.trace) {
    std::vector<unsigned long long> host(trace_n);
    NML_HIP(hipMemcpy(host.data(), pa.trace, trace_n * 8, hipMemcpyDeviceToHost));
    FILE* fp = std::fopen(trace_path, "wb");
    NML_REQUIRE(fp != nullptr, "cannot write %s", trace_path);
    const int hdr[3] = {kPersistGroups, persist_trace_stride(m->L), m->L};
    std::fwrite(hdr, sizeof(hdr), 1, fp);
    std::fwrite(host.data(), 8, trace_n, fp);
    std::fclose(fp);
  }
  NML_REQUIRE((herr & 4) == 0, "persistent decode: a data exchange timed out");
  NML_REQUIRE(herr == 0, "Token ID out of range [0, %d)", m->V);
  return 0;
}

int nml_model_last_decode_ms(nml_model* m, float* ms_per_step) {
  NML_REQUIRE(m != nullptr, "model is null");
  *ms_per_step = m->last_decode_steps > 0 ? m->last_decode_ms / m->last_decode_steps : 0.f;
  return 0;
}

int nml_model_last_decode_path(nml_model* m, int* persistent) {
  NML_REQUIRE(m != nullptr, "model is null");
  *persistent = m->last_decode_persistent;
  return 0;
}

}  // extern "C"
