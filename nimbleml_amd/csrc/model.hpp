// The model object shared by the inference driver (model.hip) and the training driver
// (train.hip): device-resident parameters in one arena, the workspaces, and the
// parameter-slot helpers.
#pragma once

#include <vector>

#include "kernels.hpp"
#include "nimbleml_hip.h"

namespace nml {

constexpr float kEps = 1e-5f;  // RMSNorm epsilon (layers/rms_norm.py:16)

struct Layer {
  void *ln1, *wqkv, *bqkv, *wo, *bo, *ln2, *w1, *b1, *w2, *b2;
};

// A grow-only device buffer.
struct Buf {
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
  void release() {
    if (p) (void)hipFree(p);
    p = nullptr;
    bytes = 0;
  }
};

inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

struct TrainState;  // train.hip: saved activations and gradients

}  // namespace nml

struct nml_model {
  int V, d, H, L, P, F, dt, dk;
  size_t es;
  void* arena = nullptr;
  size_t arena_bytes = 0;
  void *emb = nullptr, *pos = nullptr, *lnf = nullptr;
  // rotary positions (GPT(use_rope=True)): (P, dk/2) cos and sin tables; on once both set
  void *rope_cos = nullptr, *rope_sin = nullptr;
  bool rope_cos_set = false, rope_sin_set = false;
  std::vector<nml::Layer> layers;
  nml::Buf ws;         // activations
  nml::Buf ws2;        // activations of the second half of a split batched decode
  nml::Buf kvs;        // K/V scratch for forward() without a cache
  nml::Buf logits_ws;  // logits chunk for compute_loss / generate
  nml::Buf small;      // device counters, positions, loss accumulators
  nml::Buf persist;    // persistent decode: layer pointer table, exchange slots, epoch
  nml::Buf ragged;     // packed ragged prefill: row table, lengths, row starts
  nml::TrainState* train = nullptr;  // gradients and saved activations, once enabled
  // decode timing of the last generate()
  float last_decode_ms = 0.f;
  int last_decode_steps = 0;
  int last_decode_persistent = 0;
};

namespace nml {

size_t param_elems(const nml_model* m, int kind);
void** param_slot(nml_model* m, int kind, int layer);

extern const int kLayerKinds[10];

inline bool rope_on(const nml_model* m) { return m->rope_cos_set && m->rope_sin_set; }

// Learned position table for the embedding; none with rotary positions.
inline const void* posw(const nml_model* m) { return rope_on(m) ? nullptr : m->pos; }

int check_ready(nml_model* m);

// Training state teardown (train.hip), called by nml_model_destroy.
void train_release(nml_model* m);
// After a parameter upload: an fp16 model's AdamW master copy of that parameter (when the
// optimizer state exists) is taken again from the uploaded values.
int train_param_uploaded(nml_model* m, const void* param, size_t elems);

}  // namespace nml
