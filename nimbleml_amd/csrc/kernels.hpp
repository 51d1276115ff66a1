// Internal launch interface between the kernel files and the model driver.
// All launches are asynchronous on the library stream; each returns 0 or -1
// (with the message set through nml::set_error).
#pragma once

#include "common.hpp"

namespace nml {

// Epilogues of the projection kernels (x · Wᵀ, fp32 accumulation). "T(v)"
// rounds to the storage type, reproducing the reference's separate NumPy ops
// (`x @ w`, then `+ b`, then GELU / residual add: neural_network/_fused_arrays.py
// :25-30, :69-71, :200-205, :262, :270).
enum Epilogue : int {
  EPI_NONE = 0,        // out = T(acc)
  EPI_BIAS = 1,        // out = T(T(acc) + b)
  EPI_BIAS_GELU = 2,   // out = gelu_T(T(T(acc) + b))
  EPI_BIAS_RESID = 3,  // out = T(r + T(T(acc) + b))
  EPI_QKV = 4,         // T(T(acc) + b) scattered to head-major Q and the K/V cache
  EPI_CE = 5,          // fp16 tied head fused with cross-entropy: softmax partials, no output
};

// Destination of the QKV epilogue. Output row r = b·S + s of the projection is
// token s of sequence b, at absolute position pos(b) + s where pos(b) is
// pos_base[b] (device) or 0 when pos_base is null. Column n selects
// q/k/v = n / d, head h = (n % d) / dk, lane j = n % dk.
//   q  : [(b·H + h)·S + s]·dk + j                       (head-major, per call)
//   k,v: b·kv_stride_b + h·kv_stride_h + pos·dk + j     (cache layout)
struct QKVDst {
  void* q;
  void* k;
  void* v;
  const int32_t* pos_base;
  long long kv_stride_b;
  long long kv_stride_h;
  int S, H, dk, d;
  // Packed ragged rows: row m is position s of sequence b, row_seg[m] = (b << 16) | s
  // (s < 65536); q keeps the padded (B, H, S, dk) layout. Null: b = m / S, s = m % S.
  const int32_t* row_seg;
};

// Destination of the EPI_CE epilogue (fp16, 256 × 256 tiles): for row m and column tile
// t (256 columns), part[m·tiles_n + t] = (mx, Σ rnd(exp(rnd(x − mx)))) over the tile's
// fp16 logits x (mx their maximum; the terms rounded where ce_rows rounds them), and
// label_logit[m] = the fp16 logit of column labels[m], written by the tile holding it.
// The logits themselves are never stored.
struct CEDst {
  const int64_t* labels;
  float2* part;
  float* label_logit;
  int tiles_n;
};

struct LinearArgs {
  const void* x;     // (M, K) rows at stride lda
  long long lda;
  const void* w;     // (N, K) row-major: the reference's (in, out) weight transposed
  const void* bias;  // (N) or null for EPI_NONE
  const void* resid; // (M, N) for EPI_BIAS_RESID (may alias out)
  void* out;         // (M, N) row-major, ldc = N
  int M, N, K;
  int epi;
  QKVDst qkv;
  // Decode fusion of RMSNorm into the fp16 skinny GEMM (linear_norm_fusable): x is
  // normalised on load, gain norm_g (K values), from ssq_in = per-row sums of squares
  // of x in 16-column pieces, laid out (M, K/16); and an EPI_BIAS_RESID GEMM writes
  // the same sums of its output to ssq_out, (M, N/16). Null: not used.
  const float* ssq_in;
  const void* norm_g;
  float norm_eps;
  float* ssq_out;
  // EPI_BIAS_GELU with more than 64 rows: also writes the pre-activation x·Wᵀ + b, (M, N),
  // the value the GELU was taken of (the training forward keeps it). Null: not written.
  void* pre_out;
  CEDst ce;  // EPI_CE only
};

// Whether launch_linear can fuse RMSNorm into this GEMM (ssq_in / ssq_out above).
bool linear_norm_fusable(int dt, int M, int K, int N);
// Whether launch_linear takes EPI_CE for this shape (x 16-byte aligned, lda = K); the
// column tile width of its partials is kLinearCETile.
bool linear_ce_fusable(int dt, int M, int K, int N);
constexpr int kLinearCETile = 256;

int launch_linear(int dt, const LinearArgs& a, hipStream_t st);
// Workspace of the split-K skinny GEMM (8 < M ≤ 64) for outputs up to max_n wide.
// Without it (or when too small) that GEMM runs unsplit. Call outside stream capture.
int linear_reserve_workspace(int max_n);

int launch_embed(int dt, const int64_t* ids, const void* emb, const void* pos,
                 const int32_t* pos_base, void* out, int B, int S, int d, int V, int P,
                 int* err, hipStream_t st);
// Decode: row b embeds tokens[b·tok_stride + pos[b]] at position pos[b].
int launch_embed_decode(int dt, const int64_t* tokens, long long tok_stride, const int32_t* pos,
                        const void* emb, const void* posw, void* out, int B, int d, int V, int P,
                        int* err, hipStream_t st);

// Rotary positions on q (B, H, S, dk) and the K rows just written to the cache, in place
// (utils/rope.py:22-44, GPT-NeoX half split): row s of sequence b sits at position
// pos_base[b] + s (pos_base null → s); rows s ≥ seq_len[b] are skipped when seq_len is
// given. cos/sin: (max_len, dk/2) in the compute dtype.
int launch_rope(int dt, void* q, void* k, long long kv_stride_b, long long kv_stride_h, int B,
                int H, int S, int dk, const int32_t* pos_base, const int32_t* seq_len,
                const void* cos, const void* sin, int max_len, hipStream_t st);

int launch_rmsnorm(int dt, const void* x, const void* g, void* out, float* ms, float* rms,
                   int rows, int d, float eps, hipStream_t st);
int launch_gelu(int dt, const void* x, void* out, float* tanh_u, size_t n, hipStream_t st);

// Causal attention for S new queries per sequence. q is head-major
// (B, H, S, dk); keys/values at positions [0, pos(b) + S) are read from
// k/v at b·kv_stride_b + h·kv_stride_h + p·dk; query s sits at pos(b) + s and sees
// keys p ≤ pos(b) + s. Output is merged-head (B·S, H·dk).
// Largest head dim the attention kernels take (the reference's device flash kernel
// accepts dk ≤ 256, native/src/sdpa_cuda.cu:237).
constexpr int kMaxHeadDim = 256;

struct AttnArgs {
  const void* q;
  const void* k;
  const void* v;
  void* out;
  const int32_t* pos_base;  // null → 0
  long long kv_stride_b, kv_stride_h;
  int B, H, S, dk;
  float scale;  // the reference's sqrt(dk) divisor (attention.py:135)
  // Ragged prefill: sequence b has seq_len[b] ≤ S queries (q stays padded to S per
  // (b, head)) and its output rows start at row_start[b]. Null: S each, rows b·S + s.
  const int32_t* seq_len;
  const int32_t* row_start;
  // Training: per (sequence, head, query) log Σ exp(score − max) + max of the softmax,
  // (B, H, S) floats (float32 models only). Null: not written.
  float* lse;
  // The same row's max score and Σ exp(score − max) separately, (B, H, S) floats (the
  // m and l of the reference's flash kernel, sdpa_cuda.cu:40-77). Null: not written.
  float* m_out;
  float* l_out;
  // Non-causal attention (full != 0): every query sees all S keys, with mask[s·S + key]
  // (an additive (S, S) matrix in the compute dtype) added to each scaled score when
  // mask is non-null — the dense path of kernels/fused_sdpa.py:71-78. Dense rows only
  // (no pos_base, no ragged rows). Zero: causal.
  int full;
  const void* mask;
};
int launch_attention_prefill(int dt, const AttnArgs& a, hipStream_t st);

// One new query per sequence at position pos[b] (keys 0..pos[b]). `ws` is a workspace
// of attention_decode_workspace(B, H, dk, max_len) bytes, zeroed once before the first
// launch (outside stream capture); each launch leaves it zeroed again. `max_len`
// bounds pos[b] + 1.
int launch_attention_decode(int dt, const AttnArgs& a, const int32_t* pos, int max_len,
                            void* ws, hipStream_t st);
size_t attention_decode_workspace(int B, int H, int dk, int max_len);

// Row-wise cross-entropy over (rows, V) logits of storage type T. Writes the
// per-row loss (rows) and a validity flag (0 for ignore_index rows).
int launch_ce_rows(int dt, const void* logits, int rows, int V, const int64_t* labels,
                   long long ignore_index, int has_ignore, float* row_loss, int* row_valid,
                   int* err, hipStream_t st);
// Per-row loss from the EPI_CE partials (tiles_n per row): lse = M + log(Σ_t s_t·
// exp(mx_t − M)), M = max_t mx_t, loss = lse − label_logit; row flags as launch_ce_rows.
int launch_ce_combine(const float2* part, int tiles_n, const float* label_logit, int rows, int V,
                      const int64_t* labels, long long ignore_index, int has_ignore,
                      float* row_loss, int* row_valid, int* err, hipStream_t st);
// Sum of valid row losses / count → out[0] (double); 0 when no row is valid.
int launch_ce_reduce(const float* row_loss, const int* row_valid, int rows, double* sum_count,
                     int accumulate, hipStream_t st);
int launch_ce_finalize(const double* sum_count, double* loss, hipStream_t st);

// Next-token selection over (B, V) logits, models/generate.py:23-59 semantics.
struct SampleArgs {
  const void* logits;       // (B, V) storage type
  long long logits_stride;  // elements between rows
  int B, V;
  float temperature;        // ≤ 0 → greedy argmax
  int top_k;                // ≤ 0 → off
  float top_p;              // outside (0,1) → off
  float rep_penalty;        // 1 → off
  const double* uniforms;   // uniforms[step·B + b]; step = pos[b] + 1 − plen[b]
  int64_t* tokens;          // (B, tok_stride) token history of each row
  long long tok_stride;
  // Generation mode (pos non-null): the history is tokens[b][0..pos[b]]; the choice
  // is written to tokens[b][pos[b] + 1], pos[b] advances by one, and the uniform is
  // uniforms[(pos[b] + 1 − plen[b])·B + b].
  int32_t* pos;
  const int32_t* plen;
  // Standalone mode (pos null): history tokens[b][0..hist_len[b]) (null → empty),
  // uniform uniforms[b], nothing but out_ids is written.
  const int32_t* hist_len;
  int64_t* out_ids;         // optional (B) copy of the chosen ids
};
int launch_sample(int dt, const SampleArgs& a, hipStream_t st);

// ------------------------------------------------------------ training
// Every launch takes the model's storage type dt (F32 or F16) for the activation-side
// tensors; parameter gradients, partial sums and the softmax statistics are float32.
//
// General GEMM of the backward pass: C(m, n) = Σ_k A(m, k)·B(n, k), A(m, k) = a[m·lda + k]
// when a_kc (k contiguous) else a[k·lda + m]; B(n, k) likewise with b, ldb, b_kc; operands
// of type dt, fp32 products and sums. C is row-major at ldc: GB_SET stores dt, GB_ADD adds
// fp32(dt(acc)) to an fp32 C (gradient accumulation), GB_GELU stores dt(dt(acc)·gelu'(aux))
// with aux the pre-activation (dt) at ldaux.
struct GemmBwdArgs {
  const void* a;
  long long lda;
  const void* b;
  long long ldb;
  void* c;
  long long ldc;
  const void* aux;
  long long ldaux;
  int M, N, K;
};
enum GemmBwdOut : int { GB_SET = 0, GB_ADD = 1, GB_GELU = 2 };
int launch_gemm_bwd(int dt, const GemmBwdArgs& g, bool a_kc, bool b_kc, int out, hipStream_t st);

// RMSNorm backward over rows × d (kernels/fused_rmsnorm.py:195-217): dx = result, or
// dx += result when acc; dgamma (fp32) += Σ_rows dy·x̂. part: scratch of
// rmsnorm_bwd_parts(rows) · d floats.
int rmsnorm_bwd_parts(int rows);
int launch_rmsnorm_bwd(int dt, const void* dy, const void* x, const void* gamma, void* dx, int acc,
                       float* dgamma, float* part, int rows, int d, float eps, hipStream_t st);
// out[n] (fp32) += Σ_rows a[r·lda + n] (bias gradients); part: colsum_parts(rows) · n floats.
int colsum_parts(int rows);
int launch_colsum(int dt, const void* a, long long lda, int rows, int n, float* out, float* part,
                  hipStream_t st);
// In place: logits rows → (softmax − onehot(label))·scale, ignored rows → 0
// (kernels/fused_crossentropy.py:33-50).
int launch_ce_grad(int dt, void* logits, int rows, int V, const int64_t* labels,
                   long long ignore_index, int has_ignore, float scale, hipStream_t st);

// Attention backward for one layer (kernels/fused_sdpa.py:26-29, :81-88). q, k, v
// head-major (B, H, S, dk) as the forward saw them (after RoPE); o and dout merged-head
// (B·S, H·dk); lse from the forward; dvec scratch (B, H, S) floats. Writes dq, dk, dv
// into dqkv (B·S, 3·H·dk) at column offsets 0, H·dk, 2·H·dk (all of type dt). Causal
// unless `full`; a full call may add an (S, S) mask of type dt to the scores, as the
// forward's non-causal path did (the scalar kernels take it).
struct AttnBwdArgs {
  const void* q;
  const void* k;
  const void* v;
  const void* o;
  const void* dout;
  const float* lse;
  float* dvec;
  void* dqkv;
  int B, H, S, dk;
  float scale;  // sqrt(dk), the divisor of the scores
  int full = 0;
  const void* mask = nullptr;
};
int launch_attention_backward(int dt, const AttnBwdArgs& a, hipStream_t st);
// RoPE backward on dqkv rows (the dq and dk parts): pair (i, i + dk/2) of row b·S + s
// rotated by −θ at position s (cos/sin: (max_len, dk/2) of type dt).
int launch_rope_backward(int dt, void* dqkv, int rows, int S, int H, int dk, const void* cos,
                         const void* sin, hipStream_t st);
// Embedding backward: dE[ids[r]] += g[r] (token rows), dpos[s] += Σ_b g[b·S + s]
// (dpos null: none); g of type dt, dE and dpos fp32.
int launch_embed_backward(int dt, const void* g, const int64_t* ids, float* demb, float* dpos, int B,
                          int S, int d, int V, hipStream_t st);

// Elementwise dtype conversion (F16 → F32 or F32 → F16, round to nearest even).
int launch_convert(int src_dt, const void* src, int dst_dt, void* dst, size_t n, hipStream_t st);

// AdamW over n float32 elements in place (native/src/adamw.cpp:6-20 operation order);
// buffers 16-byte aligned.
int launch_adamw(float* p, const float* g, float* m, float* v, size_t n, float lr, float beta1,
                 float beta2, float bias1, float bias2, float eps, float weight_decay,
                 hipStream_t st, void* p16 = nullptr);

// Persistent decode step (batch 1): one launch of kPersistGroups workgroups runs the
// whole token; see decode_persist.hip.
constexpr int kPersistGroups = 256;
constexpr int kPersistMaxLen = 2048;  // attention length bound (max_seq_len)

struct PersistArgs {
  // Parameters of layer 0; layer l's are at + l·layer_bytes (one arena, same layout
  // per layer), so no pointer has to be loaded from memory inside the kernel.
  const void *ln1, *wqkv, *bqkv, *wo, *bo, *ln2, *w1, *b1, *w2, *b2;
  long long layer_bytes;
  const void* emb;
  const void* posw;
  const void* lnf;
  void* kc;                    // K cache of layer 0; layer l at + l·kv_layer elements
  void* vc;
  long long kv_layer, kv_head; // elements between layers / heads
  int64_t* tokens;             // token history of the row; tokens[pos] is fed
  int32_t* pos;                // pos[0]: position of the fed token (advanced when fused)
  void* logits;                // (V) logits of the step
  unsigned long long* slots;   // exchange slots, persist_slot_count() entries, zeroed
  uint32_t* epoch;             // step counter, ≥ 1, advanced by the kernel
  int* err;                    // bit 0: token/position out of range; bit 2: exchange timeout
  int V, L, P;
  int fuse_argmax;             // greedy: write tokens[pos+1] and advance pos in-kernel
  float scale;                 // sqrt(dk)
  // Optional phase timestamps (wall_clock64) of each workgroup: trace[g·stride + mark],
  // stride = persist_trace_stride(L), and at mark 2 the workgroup's XCD. Null: no tracing.
  unsigned long long* trace;
};

// Marks: 0 start, 1 embedded; layer l at 4 + kMarks·l + {0 P1 loads issued, 1 x in,
// 2 QKV out, 3 q in, 4 chunks out, 5 merged, 6 attention in, 7 x_mid in, 8 h in,
// 9 x out, 10 x_mid out, 11 W1 loads issued, 12 h out, 13 W2 loads issued, 14 K/V
// loads issued, 15 W_o loads issued}; head at 4 + kMarks·L + {0 x in, 1 logits out,
// 2 choice}.
constexpr int kMarks = 16;
__host__ __device__ inline int persist_trace_stride(int L) { return 4 + kMarks * L + 4; }

bool persist_supported(int dt, int d, int H, int F, int B, int P);
size_t persist_slot_count(int d, int H);
int launch_decode_persist(int dt, int d, int H, const PersistArgs& a, hipStream_t st);

}  // namespace nml
