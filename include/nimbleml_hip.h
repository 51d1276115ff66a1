/* nimbleml_hip.h — C-ABI of the MI355X (gfx950) GPT token-loop library.
 *
 * The drop-in boundary for NimbleML's GPT path (prefill → decode, compute_loss).
 * Conventions follow the reference extension's device-pointer API
 * (native/src/module.cpp:229-285): the caller owns every input/output buffer and
 * passes plain device pointers and sizes; launches are asynchronous on the
 * library stream; failures are reported instead of thrown — every function
 * returns 0 on success or -1, and nml_last_error() gives the message (the
 * reference raises RuntimeError with the CUDA message, sdpa_cuda.cu:10-14).
 *
 * dtype arguments: 0 = float32, 1 = float16 (NIMBLEML_DTYPE, np_backend.py:157-176).
 * Token ids and labels are int64 (Tensor.from_int64, utils/tensor.py:194-214).
 */
#ifndef NIMBLEML_HIP_H
#define NIMBLEML_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------------------------------------------------------- runtime ---- */

/* Capability probes; replace `with_cuda` (module.cpp:13-17) and
 * `flash_sdpa_available()` (module.cpp:221-227). */
int nml_with_hip(void);
int nml_hip_available(int* device_count);
const char* nml_last_error(void);

/* Select the device and create the library stream (default priority). */
int nml_init(int device);
int nml_get_stream(void** stream);
int nml_set_stream(void* stream);
int nml_device_info(char* name, size_t name_len, int* cu_count, size_t* total_mem);

/* Device memory. Replace CuPy's allocator for this path (np_backend.py:82-90). */
int nml_malloc(size_t bytes, void** ptr);
int nml_free(void* ptr);
int nml_memcpy_h2d(void* dst, const void* src, size_t bytes); /* returns when done */
int nml_memcpy_d2h(void* dst, const void* src, size_t bytes); /* returns when done */
int nml_memcpy_d2d(void* dst, const void* src, size_t bytes); /* async */
int nml_memset(void* dst, int value, size_t bytes);            /* async */
int nml_synchronize(void); /* replaces sync_device(), np_backend.py:118-126 */

/* Events on the library stream (timing). */
int nml_event_create(void** ev);
int nml_event_record(void* ev);
int nml_event_elapsed_ms(void* start, void* end, float* ms);
int nml_event_destroy(void* ev);

/* ------------------------------------------------------------ single ops ---- */

/* RMSNorm forward; same arguments as rmsnorm_forward_device (module.cpp:259-270,
 * kernel sdpa_cuda.cu:135-165) plus dtype. ms/rms (float32, rows) may be NULL.
 * Semantics: kernels/fused_rmsnorm.py:153-162 (fp16 branch :153-158). */
int nml_rmsnorm_forward_device(const void* x, const void* gamma, void* out, float* ms,
                               float* rms, size_t rows, size_t dim, float eps, int dtype);

/* tanh-GELU forward; replaces gelu_forward (module.cpp:19-31, native/src/gelu.cpp:12-21)
 * and the fp16 NumPy branch (kernels/fused_gelu.py:67-69). tanh_u may be NULL. */
int nml_gelu_forward_device(const void* x, void* out, float* tanh_u, size_t n, int dtype);

/* x[b,s] = weights[ids[b,s]] + pos_weights[pos_offsets[b] + s] (pos_offsets NULL → 0).
 * Replaces embedding_lookup + forward_prefix (kernels/embedding_scatter.py:25-36,
 * layers/embedding.py:72-118, models/gpt.py:85-86). Out-of-range ids or positions
 * write zeros and set bit 0 of *err (err may be NULL). */
int nml_embedding_gather_device(const void* weights, const void* pos_weights, const int64_t* ids,
                                void* out, size_t batch, size_t seq, size_t dim, size_t vocab,
                                size_t max_pos, const int32_t* pos_offsets, int* err, int dtype);

/* out = epi(x · w_tᵀ): x (rows, in_f) at row stride ld_x, w_t (out_f, in_f) — the
 * reference's Dense weight (in, out) (layers/dense.py:16-25) transposed.
 * epilogue: 0 none, 1 +bias, 2 +bias then GELU, 3 resid + (x·wᵀ + bias).
 * Replaces the `x @ W + b` GEMMs of neural_network/_fused_arrays.py:25-30,69-71,
 * 200-205 and the tied head `h @ Eᵀ` (models/gpt.py:150-153, with w_t = E). */
int nml_linear_device(const void* x, size_t ld_x, const void* w_t, const void* bias,
                      const void* resid, void* out, size_t rows, size_t in_f, size_t out_f,
                      int epilogue, int dtype);

/* Causal flash attention in float32 with the reference's device-pointer arguments:
 * flash_sdpa_forward_device (module.cpp:231-242 → flash_sdpa_forward_cuda,
 * sdpa_cuda.cu:40-77, 235-243), as kernels/fused_sdpa.py:91-115 calls it. q, k, v, out:
 * (bh, seq, dk); scores s_ij = (q_i·k_j)·scale for keys j ≤ i — `scale` multiplies (the
 * caller passes 1/sqrt(dk)); m, l: (bh, seq), each query row's max score and
 * Σ_j exp(s_ij − m). Any head dim 1 ≤ dk ≤ 256 (sdpa_cuda.cu:237 takes dk ≤ 256). */
int nml_flash_sdpa_forward_device(const float* q, const float* k, const float* v, float* out,
                                  float* m, float* l, size_t bh, size_t seq, size_t dk,
                                  float scale);
/* Its backward: flash_sdpa_backward_device (module.cpp:243-257 → flash_sdpa_backward_cuda,
 * sdpa_cuda.cu:79-133, 245-256). grad_out, q, k, v, grad_q/k/v: (bh, seq, dk); m, l from the
 * forward; grad_q, grad_k, grad_v are overwritten. */
int nml_flash_sdpa_backward_device(const float* grad_out, const float* q, const float* k,
                                   const float* v, const float* m, const float* l, float* grad_q,
                                   float* grad_k, float* grad_v, size_t bh, size_t seq, size_t dk,
                                   float scale);
/* RMSNorm backward in float32: rmsnorm_backward_device (module.cpp:271-284 →
 * rmsnorm_backward_cuda, sdpa_cuda.cu:167-201, 225-233). grad, x, grad_x: (rows, dim);
 * grad_x and grad_gamma (dim) are overwritten. ms/rms (the forward's statistics) may be
 * NULL: they are recomputed from x. */
int nml_rmsnorm_backward_device(const float* grad, const float* x, const float* gamma,
                                const float* ms, const float* rms, float* grad_x,
                                float* grad_gamma, size_t rows, size_t dim, float eps);

/* Backward helpers of the module-level autograd closures, in the compute dtype (dtype 0
 * float32, 1 float16); parameter gradients are float32 and ADDED to, as
 * Tensor._accumulate_grad does (utils/tensor.py:334-352). Each returns after the device
 * finishes. */
/* Dense.forward's closure (layers/dense.py:81-94): dy (rows, out), x (rows, in), w_t the
 * weight transposed to (out, in), as the device keeps it. dx (rows, in) = dy·W is
 * overwritten; with gelu_pre (rows, in) non-NULL — the pre-activation whose GELU gave x —
 * dx = (dy·W)·gelu'(gelu_pre) instead, the GELU backward of FeedForward's closure
 * (neural_network/feed_forward.py:105-129, kernels/fused_gelu.py:86-111). dw_t
 * (out, in) += dyᵀ·x; db (out) += Σ_rows dy. dx, dw_t, db may each be NULL. */
int nml_linear_backward_device(const void* dy, const void* x, const void* w_t, void* dx,
                               float* dw_t, float* db, size_t rows, size_t in_features,
                               size_t out_features, const void* gelu_pre, int dtype);
/* RMSNorm's closure (layers/rms_norm.py:76-94 → kernels/fused_rmsnorm.py:195-217) in the
 * compute dtype: grad_x (rows, dim) overwritten, grad_gamma (dim, float32) added to. */
int nml_rmsnorm_backward_typed_device(const void* grad, const void* x, const void* gamma,
                                      void* grad_x, float* grad_gamma, size_t rows, size_t dim,
                                      float eps, int dtype);
/* Embedding's closure (layers/embedding.py:63-69 → kernels/embedding_scatter.py:39-60):
 * grad_weights[ids[r]] += grad[r] for each of the rows, in ascending row order per id;
 * ids outside [0, vocab) add nothing. */
int nml_embedding_backward_device(const void* grad, const int64_t* ids, float* grad_weights,
                                  size_t rows, size_t dim, size_t vocab, int dtype);

/* Causal attention in the compute dtype as the reference's CPU path computes it for GPT
 * (kernels/fused_sdpa.py:71-78, reached from fused_sdpa_forward :256-289 with the causal
 * mask): scores (q·k) / scale_div with scale_div = sqrt(dk) (attention.py:135), softmax,
 * then P·v. q, k, v, out: (bh, seq, dk). */
int nml_causal_attention_device(const void* q, const void* k, const void* v, void* out, size_t bh,
                                size_t seq, size_t dk, float scale_div, int dtype);

/* fused_sdpa_forward for any mask (kernels/fused_sdpa.py:256-289 → _matmul_sdpa_forward
 * :71-78): causal != 0 is the causal case above (mask must be NULL); causal == 0 attends
 * every query to all seq keys, adding mask[i·seq + j] (an additive (seq, seq) matrix in
 * the compute dtype, e.g. 0 / −inf) to each scaled score when mask is non-NULL, and to
 * nothing when it is NULL (the reference's mask_arr=None). */
int nml_sdpa_forward_device(const void* q, const void* k, const void* v, const void* mask,
                            void* out, size_t bh, size_t seq, size_t dk, float scale_div,
                            int causal, int dtype);

/* One new query per (row, head) against a KV cache: the attention of a decode step behind
 * the forward_with_cache(ids, cache) seam that generate() probes for
 * (models/generate.py:93-100), with the scores of kernels/fused_sdpa.py:71-78:
 * s_j = (q·k_j) / scale_div (scale_div = sqrt(dk), attention.py:135), softmax over keys
 * 0 ≤ j < lens[b], then Σ_j p_j·v_j. The reference has no KV cache and no such kernel; it
 * re-forwards the whole sequence per token (generate.py:101-103).
 *   q:      (batch, heads, dk) — the new token's query of each row
 *   kcache, vcache: (batch, heads, max_seq, dk) — one head's keys are contiguous
 *   lens:   device int32 (batch): keys attended per row, 1 ≤ lens[b] ≤ max_seq; a length
 *           outside that range is clamped into it and sets bit 0 of *err (err: device int,
 *           may be NULL; the caller clears it)
 *   out:    (batch, heads·dk) — merged heads, as the W_o projection reads them
 * Any head dim 1 ≤ dk ≤ 256; float32 or float16 (dtype). Asynchronous on the library
 * stream; the library keeps a grow-only workspace (allocated and cleared on the first call
 * at a larger shape, so do not capture that call into a graph). */
int nml_decode_attention_device(const void* q, const void* kcache, const void* vcache,
                                const int32_t* lens, void* out, size_t batch, size_t heads,
                                size_t max_seq, size_t dk, float scale_div, int* err, int dtype);

/* Mean tied-head cross-entropy (kernels/fused_tied_crossentropy.py:8-24 →
 * fused_crossentropy.py:14-30) without materialising all (rows, vocab) logits at once.
 * has_ignore: drop rows with label == ignore_index (losses/_ce_prepare.py:46-69).
 * *loss receives the mean as float64 (returns after the device finishes). */
int nml_tied_ce_forward_device(const void* hidden, const void* weights, const int64_t* labels,
                               size_t rows, size_t dim, size_t vocab, int64_t ignore_index,
                               int has_ignore, double* loss, int dtype);

/* nml_tied_ce_forward_device without any device allocation: no counterpart in the
 * reference. For callers that cannot allocate device memory (tight serving or training
 * loops, harnesses that forbid hipMalloc). The logits chunks live in a fixed 32 MiB
 * device scratch that the library holds on each GPU it runs on, so rows go through in
 * chunks of at most 32 MiB / (vocab · element size) rows; a vocabulary whose single row
 * does not fit is refused with an error. Same arguments and result as
 * nml_tied_ce_forward_device; calls on one GPU share the scratch, so they must not
 * overlap (one stream, or synchronise between them). */
int nml_tied_ce_forward_device_noalloc(const void* hidden, const void* weights,
                                       const int64_t* labels, size_t rows, size_t dim,
                                       size_t vocab, int64_t ignore_index, int has_ignore,
                                       double* loss, int dtype);

/* Next-token choice per row of (batch, vocab) logits (models/generate.py:23-59):
 * temperature ≤ 0 → argmax; else temperature, top_k (≤0 off), top_p (outside (0,1) off)
 * with u[b] replacing RandomState.choice's draw. repetition_penalty uses
 * history[b, 0:hist_len[b]] (history/hist_len may be NULL when the penalty is 1). */
int nml_sample_device(const void* logits, size_t batch, size_t vocab, float temperature,
                      int top_k, float top_p, float repetition_penalty, const double* u,
                      const int64_t* history, size_t history_stride, const int32_t* hist_len,
                      int64_t* out_ids, int dtype);

/* Optimizer step, float32 state, in place on device buffers.
 * adamw_step (native/src/module.cpp:175-188 → adamw_step_cpu, native/src/adamw.cpp:6-20):
 * the same operation order, so results equal the reference's bit for bit. n elements;
 * all four buffers 16-byte aligned. */
int nml_adamw_step_device(float* param, const float* grad, float* m, float* v, size_t n, float lr,
                          float beta1, float beta2, float bias1, float bias2, float eps,
                          float weight_decay);
/* clip_grad_norm (module.cpp:190-200 → clip_grad_norm_cpu, adamw.cpp:22-37): the global L2
 * norm of n_tensors gradients (device pointers in a host array, element counts in sizes),
 * accumulated in float64; when it exceeds max_norm every gradient is scaled by
 * max_norm / (norm + 1e-6). Writes the norm (float) to *norm; returns when done. */
int nml_clip_grad_norm_device(float* const* grads, const size_t* sizes, size_t n_tensors,
                              float max_norm, float* norm);

/* ------------------------------------------------------------ GPT model ---- */

/* Parameter kinds for nml_model_set_param. Host data must already be in device
 * layout and dtype: Dense weights transposed to (out, in); Q/K/V stacked. */
enum nml_param_kind {
  NML_P_TOKEN_EMB = 0, /* (vocab, d)        token_emb.weights            */
  NML_P_POS_EMB = 1,   /* (max_seq, d)      pos_emb.weights              */
  NML_P_LN_F = 2,      /* (d)               ln.gamma                     */
  NML_P_ROPE_COS = 3,  /* (max_seq, dk/2)   cos(p·θ_i), utils/rope.py:12-19, in the compute
                        *                   dtype as apply_rope_flat casts it (:37-38)   */
  NML_P_ROPE_SIN = 4,  /* (max_seq, dk/2)   sin(p·θ_i); once both are set the model uses
                        *                   rotary positions (GPT(use_rope=True),
                        *                   models/gpt.py:46-51) and ignores pos_emb     */
  NML_P_LN1 = 10,      /* (d)               blocks.layers.i.ln1.gamma    */
  NML_P_WQKV = 11,     /* (3d, d)           [W_q | W_k | W_v]ᵀ           */
  NML_P_BQKV = 12,     /* (3d)              [b_q | b_k | b_v]            */
  NML_P_WO = 13,       /* (d, d)            W_oᵀ                         */
  NML_P_BO = 14,       /* (d)                                            */
  NML_P_LN2 = 15,      /* (d)               ln2.gamma                    */
  NML_P_W1 = 16,       /* (d_ff, d)         ffn.dense1.weightsᵀ          */
  NML_P_B1 = 17,       /* (d_ff)                                         */
  NML_P_W2 = 18,       /* (d, d_ff)         ffn.dense2.weightsᵀ          */
  NML_P_B2 = 19        /* (d)                                            */
};

typedef struct nml_model nml_model;
typedef struct nml_cache nml_cache;

/* A GPT of the reference's architecture (models/gpt.py:11-71, fused_blocks=True,
 * absolute learned positions): device-resident parameters in one allocation. */
int nml_model_create(int vocab, int d_model, int num_heads, int num_layers, int max_seq_len,
                     int d_ff, int dtype, nml_model** out);
int nml_model_destroy(nml_model* m);
int nml_model_set_param(nml_model* m, int kind, int layer, const void* host, size_t bytes);
/* Device pointer of a parameter (for tests). */
int nml_model_param_ptr(nml_model* m, int kind, int layer, void** ptr);

/* GPT.forward (models/gpt.py:92-121): logits (batch, seq, vocab); last_only → (batch, vocab)
 * for the last position. ids: device int64 (batch, seq). */
int nml_model_forward(nml_model* m, const int64_t* ids, size_t batch, size_t seq, void* logits,
                      int last_only);

/* The model's blocks over an already-embedded input: FusedTransformerBlock.forward
 * (neural_network/transformer_fused.py:44-95 → fused_block_forward_arrays,
 * _fused_arrays.py:251-284) for each layer in order, then, when final_norm != 0, the
 * final RMSNorm — FusedGPTTrunk.forward (transformer_fused.py:103-144 →
 * fused_trunk_forward_arrays). x, out: device (batch, seq, d_model) in the compute dtype
 * (they may be the same buffer); positions start at 0 (RoPE when its tables are set).
 * causal != 0 masks causally (the modules' mask=None); causal == 0 attends to every key,
 * adding mask (an additive (seq, seq) matrix, or NULL for none) to the scaled scores.
 * The token and position tables are not used. */
int nml_model_blocks_forward(nml_model* m, const void* x, void* out, size_t batch, size_t seq,
                             int final_norm, int causal, const void* mask);

/* MultiHeadAttention.forward (neural_network/attention.py:139-168) with layer `layer`'s
 * projections: out = merge(softmax(q·kᵀ / sqrt(dk) [+ mask]) · v) · W_o + b_o with
 * q, k, v = x·W_{q,k,v} + b. No rotary embedding (the module applies none). causal and
 * mask as for nml_model_blocks_forward; the module's own mask=None is causal == 0 with
 * a NULL mask. x, out: device (batch, seq, d_model), distinct buffers. */
int nml_model_mha_forward(nml_model* m, int layer, const void* x, void* out, size_t batch,
                          size_t seq, int causal, const void* mask);

/* Module-level autograd: the autograd closures that FusedTransformerBlock.forward,
 * FusedGPTTrunk.forward (neural_network/transformer_fused.py:65-78, :123-131) and the
 * attention of MultiHeadAttention.forward (neural_network/attention.py:103-119) attach.
 * A *_forward_train call computes the same output as its forward above and keeps the
 * activations its backward needs in the model's training state (one saved forward per
 * model: each saving forward, nml_model_loss_train included, replaces the last and
 * advances nml_model_saved_generation; a mask is copied). Its *_backward takes
 * dout = d(loss)/d(out) (device, the compute dtype, out's shape), ADDS d(loss)/d(param)
 * of every parameter the forward used to the float32 gradients (nml_model_grad_ptr), and
 * writes dx = d(loss)/d(x) (same shape as x; NULL skips it). Backward returns after the
 * device finishes. Non-causal and masked attention backward runs on the scalar kernels. */
int nml_model_blocks_forward_train(nml_model* m, const void* x, void* out, size_t batch,
                                   size_t seq, int final_norm, int causal, const void* mask);
/* fused_block_backward_arrays / fused_trunk_backward_arrays (_fused_arrays.py:311-377). */
int nml_model_blocks_backward(nml_model* m, const void* dout, void* dx);
int nml_model_mha_forward_train(nml_model* m, int layer, const void* x, void* out, size_t batch,
                                size_t seq, int causal, const void* mask);
/* mha_backward_arrays (_fused_arrays.py:129-184) without RoPE, the SDPA backward of
 * kernels/fused_sdpa.py:26-29, :81-88 for the forward's mask. */
int nml_model_mha_backward(nml_model* m, const void* dout, void* dx);

/* GPT.compute_loss (models/gpt.py:123-137): mean tied-head CE over batch·seq rows,
 * labels device int64. Returns after the device finishes; *loss is float64. */
int nml_model_loss(nml_model* m, const int64_t* ids, const int64_t* labels, size_t batch,
                   size_t seq, int64_t ignore_index, int has_ignore, double* loss);

/* ---- training (float32 and float16 models) -------------------------------------------
 * compute_loss with the autograd graph kept, then loss.backward() (models/gpt.py:123-137;
 * Tensor.backward, utils/tensor.py:286-332; the array-level backward of
 * neural_network/_fused_arrays.py:129-377 and kernels/fused_tied_crossentropy.py:27-48).
 * Gradients live on the device in a float32 arena laid out like the parameters: weight
 * gradients are (out, in) like the device weights, and accumulate over backward calls
 * (Tensor._accumulate_grad, utils/tensor.py:334-352) until nml_model_zero_grad. */

/* Tensor.zero_grad (utils/tensor.py:271-279) for every parameter at once; allocates the
 * gradient arena on first use. */
int nml_model_zero_grad(nml_model* m);
/* Device pointer of the float32 gradient of parameter (kind, layer), same shape as the
 * parameter (Tensor.grad). */
int nml_model_grad_ptr(nml_model* m, int kind, int layer, void** ptr);
/* GPT.compute_loss (models/gpt.py:123-137) keeping the activations its backward needs;
 * ids and labels (device int64) are copied. Same loss as nml_model_loss. */
int nml_model_loss_train(nml_model* m, const int64_t* ids, const int64_t* labels, size_t batch,
                         size_t seq, int64_t ignore_index, int has_ignore, double* loss);
/* loss.backward(grad) after nml_model_loss_train (repeatable, as with retain_graph): adds grad_scale ×
 * d(loss)/d(parameter) to every gradient (losses/cross_entropy.py:166-191, grad_scale =
 * output.grad). Returns after the device finishes. */
int nml_model_backward(nml_model* m, double grad_scale);

/* The backward of GPT.forward (models/gpt.py:92-121; its closures are the blocks' and the
 * tied head's, gpt.py:139-181, run by utils/tensor.py:286-332): recomputes the forward at
 * ids (device int64, batch × seq) keeping its activations, then ADDS d(loss)/d(parameter)
 * for dlogits = d(loss)/d(logits) (device, the compute dtype, batch × seq × vocab) to every
 * gradient. Replaces any saved forward (advances nml_model_saved_generation). Returns after
 * the device finishes. */
int nml_model_logits_backward(nml_model* m, const int64_t* ids, size_t batch, size_t seq,
                              const void* dlogits);

/* Which forward the saved activations belong to: a counter that every
 * nml_model_loss_train advances (0: nothing saved). A caller holding the loss of an
 * earlier nml_model_loss_train compares it before nml_model_backward, since backward
 * always differentiates the latest saved forward (the reference keeps one graph per loss,
 * utils/tensor.py:286-332; here the device keeps one). */
int nml_model_saved_generation(nml_model* m, unsigned long long* generation);

/* AdamW.step() over every parameter of the model (optimizers/adam.py:85-128 with the
 * native float32 update of adamw_step, native/src/adamw.cpp:6-20, in its operation order):
 * the device parameters are updated in place from the gradient arena, with first and second
 * moments kept on the device (zero before the first call). bias_corr1/2 = 1 − β^t as the
 * caller's step count gives them (adam.py:91-93). Every parameter takes weight_decay (one
 * parameter group); the rotary tables are buffers and are left alone. */
int nml_model_adamw_step(nml_model* m, float lr, float beta1, float beta2, float bias_corr1,
                         float bias_corr2, float eps, float weight_decay);
/* Device pointers of the AdamW moments of parameter (kind, layer) (the optimizer's m[i],
 * v[i], adam.py:64-83), for checkpoints and tests. */
int nml_model_adam_moments(nml_model* m, int kind, int layer, void** first, void** second);

/* Allocate the AdamW state if absent (Adam.__init__, adam.py:64-83): zero moments and,
 * for float16 models, float32 masters copied from the current parameters. Lets a
 * checkpoint's state (load_checkpoint, utils/saveload.py:334-358 → _load_optimizer_state
 * :130-175) be written through nml_model_adam_moments / nml_model_adam_master before the
 * first step. Idempotent. Parameters uploaded later with nml_model_set_param refresh their
 * masters. */
int nml_model_adam_state_init(nml_model* m);

/* Device pointer of the float32 master copy of parameter (kind, layer) of a float16 model
 * (Adam.masters[i], adam.py:75-81; saved as optimizer/master/i, saveload.py:108-110). */
int nml_model_adam_master(nml_model* m, int kind, int layer, void** master);

/* The per-parameter AdamW update of Adam._adam_update (adam.py:210-290) over elements
 * [offset, offset + count) of parameter (kind, layer) in the device layout (a contiguous
 * range: one of Q/K/V's row blocks of the stacked weight, a whole weight, a bias),
 * with that parameter group's lr and weight_decay — for optimizers whose parameter groups
 * or missing gradients (adam.py:97-104 skips parameters without one) rule out the whole-model
 * nml_model_adamw_step. offset is a multiple of 4. */
int nml_model_adamw_update(nml_model* m, int kind, int layer, size_t offset, size_t count,
                           float lr, float beta1, float beta2, float bias_corr1, float bias_corr2,
                           float eps, float weight_decay);

/* KV cache for batch rows: K and V per layer, (batch, heads, max_seq, head_dim) each.
 * The seam generate() probes for (models/generate.py:93-100). */
int nml_cache_create(nml_model* m, size_t batch, nml_cache** out);
int nml_cache_destroy(nml_cache* c);
/* The length of row 0 (rows prefilled with nml_model_prefill_ragged may differ). */
int nml_cache_length(nml_cache* c, size_t* len);
/* Append seq tokens (same count per row, each row at its own position) and return their
 * logits (batch, seq, vocab), or (batch, vocab) for the last position when last_only.
 * seq == 1 is one step of generate()'s decode loop (the same kernels as
 * nml_model_generate: the whole-step decode of the graph-launched loop); it returns
 * after the device finishes. */
int nml_model_forward_cached(nml_model* m, nml_cache* c, const int64_t* ids, size_t batch,
                             size_t seq, void* logits, int last_only);
/* Prefill an empty cache with prompts of different lengths — row b is prompts[b ·
 * prompt_stride …] of prompt_len[b] tokens (device int64; prompt_len on the host) — as
 * generate() does for a ragged batch (one packed pass); logits (batch, vocab) receive each
 * row's last-position logits. Each row then continues at its own position through
 * nml_model_forward_cached. The reference runs such rows one at a time
 * (models/generate.py:80-89); each row here gives what it gives alone. */
int nml_model_prefill_ragged(nml_model* m, nml_cache* c, const int64_t* prompts,
                             size_t prompt_stride, const int32_t* prompt_len, size_t batch,
                             void* logits);

/* Whole generate() (models/generate.py:62-119) on device, no host sync per token:
 * prompts (batch, prompt_stride) device int64, row b valid for prompt_len[b] (host array;
 * rows may differ — ragged batch); tokens_out (batch, out_stride) device int64 receives
 * prompt + max_new tokens per row. u: device float64 (max_new, batch) uniforms when
 * temperature > 0. use_graph: replay each decode step from one captured HIP graph. */
int nml_model_generate(nml_model* m, const int64_t* prompts, size_t prompt_stride,
                       const int32_t* prompt_len, size_t batch, size_t max_new,
                       float temperature, int top_k, float top_p, float repetition_penalty,
                       const double* u, int64_t* tokens_out, size_t out_stride, int use_graph);

/* Timing helper for the benchmark: average device time of one decode step
 * (embedding … sampling) over `steps` steps of the last generate() call shape. */
int nml_model_last_decode_ms(nml_model* m, float* ms_per_step);

/* Which decode step the last generate() used: 1 = the persistent one-launch-per-token
 * kernel (batch 1, d_model 1024, head_dim 64, max_seq_len ≤ 2048), 0 = one launch per
 * op. Set NIMBLEML_PERSISTENT=0 to force the latter. */
int nml_model_last_decode_path(nml_model* m, int* persistent);

#ifdef __cplusplus
}
#endif

#endif /* NIMBLEML_HIP_H */
