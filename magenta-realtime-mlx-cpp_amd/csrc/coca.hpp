// MusicCoCa text path on the device (musiccoca.cpp:118-294) and the style
// tokens StyleModel derives from it (style_model.cpp:76-121, rvq.cpp:24-62):
// prompt ids (max_text_len, BOS + SentencePiece ids, zero-padded) -> 12
// pre-norm transformer layers -> exit LayerNorm -> attention pooler ->
// 768-dim embedding -> RVQ quantisation -> style ids.  fp32 as the reference
// runs it.  The linears are the codec's implicit-GEMM matrix-core kernel
// (one 1x1 tap; bias, residual and GELU in its epilogue; split-K for the
// 128-row products); the rest are small kernels in coca_kernels.hip.
#pragma once

#include <cstdint>
#include <vector>

#include "codec.hpp"
#include "common.hpp"
#include "safetensors.hpp"

namespace mrt {

struct CocaConfig {
  int d_model = 768, num_heads = 12, d_head = 64, d_ff = 3072, num_layers = 12, pooler_d_head = 256;
  int vocab_size = 64000, max_text_len = 128, rvq_depth = 12, codebook = 1024;
};

// x (rows, D) = table[ids] * scale.
void coca_embed(const int* ids, int rows, const float* table, int vocab, int D, float scale, float* x,
                hipStream_t s);
// LayerNorm over the last axis (musiccoca.cpp:71-79): rows of D <= 4096.
void layer_norm_rows(const float* x, int rows, int D, const float* w, const float* b, float eps, float* y,
                     hipStream_t s);
// Multi-head attention core (musiccoca.cpp:155-176): q (Sq, ldq), k / v (Sk,
// ldk / ldv), head h at columns h * D; logits (q * qscale) . k / sqrt(D),
// capped cap * tanh(x / cap) when cap > 0, plus mask (Sk) when non-null,
// softmax over the keys; out (Sq, H * D).  Sk <= 256, D <= 256.
void coca_attention(const float* q, int ldq, const float* k, int ldk, const float* v, int ldv, int Sq, int Sk, int H,
                    int D, const float* qscale, float cap, const float* mask, float* out, hipStream_t s);
// rvq_quantization (rvq.cpp:24-62) of one vector (D) against codebooks (K, C,
// D), C <= 1024: tokens (K); residual (D) scratch.
void rvq_quantize(const float* vec, const float* codebooks, int K, int C, int D, float* residual, int* tokens,
                  hipStream_t s);

class Coca {
 public:
  // w: the MusicCoCa bundle (text keys); cb: the bundle holding "codebooks".
  Coca(const TensorSource& w, const TensorSource& cb, const CocaConfig& c, int device);
  ~Coca();
  Coca(const Coca&) = delete;
  Coca& operator=(const Coca&) = delete;

  const CocaConfig cfg;
  const int device;
  hipStream_t stream = nullptr;

  // MusicCoCaEncoder::embed_text for one prompt: ids / padding host
  // (max_text_len), padding 1.0 = padded; emb host (d_model) or null.  Every
  // prompt runs the same launch sequence (max_text_len rows): the first call
  // enqueues it directly, the second captures it into a HIP graph, and that
  // call and every later one replay the graph.
  void embed_text(const int32_t* ids, const float* padding, float* emb);
  // StyleModel::tokenize of the last embedding (or of `emb` when non-null):
  // tokens host (rvq_depth).
  void tokenize(const float* emb, int32_t* tokens);
  float last_ms() const;
  // Device (pointer, bytes) of an intermediate: 0 = the embedding (d_model),
  // 1 .. num_layers = layer i - 1's output (max_text_len, d_model).
  std::pair<const void*, size_t> buffer(int which) const;

 private:
  struct Lin {
    float* w = nullptr;  // (in, out_pad), packed
    float* b = nullptr;  // (out)
    int in = 0, out = 0, out_pad = 0;
  };
  struct Step {  // one GEMM launch
    ConvLaunch L;
    int tiles_m, tiles_n;
    const float* w;  // packed weights of its single sub-problem
  };
  Lin pack(const TensorSource& w, const std::vector<std::string>& names, int in);
  void enqueue_text();
  void plan_gemm(const float* x, int M, const Lin& l, float* y, const float* res, int act);
  float* dalloc(size_t floats);

  std::vector<void*> allocs_;
  float* emb_table_ = nullptr;
  std::vector<Lin> qkv_, o_, w1_, w2_;
  std::vector<float*> ln1w_, ln1b_, ln2w_, ln2b_;
  float *exit_w_, *exit_b_, *pln_w_, *pln_b_, *pquery_, *pscale_;
  Lin pq_, pkv_, po_;
  float* codebooks_ = nullptr;
  // activations
  int* ids_ = nullptr;
  float *mask_ = nullptr, *x_ = nullptr, *h_ = nullptr, *qkv_buf_ = nullptr, *att_ = nullptr, *y_ = nullptr,
        *f_ = nullptr, *n_ = nullptr, *pq_buf_ = nullptr, *pkv_buf_ = nullptr, *patt_ = nullptr, *emb_ = nullptr,
        *res_ = nullptr;
  std::vector<float*> layer_out_;
  int* tok_ = nullptr;
  int32_t* h_stage_ = nullptr;
  std::vector<Step> steps_;  // every GEMM of embed_text, in order
  ConvSub* subs_dev_ = nullptr;
  float* partial_ = nullptr;
  hipEvent_t ev_[2] = {nullptr, nullptr};
  bool timed_ = false;
  int calls_ = 0;  // embed_text calls so far
  hipGraph_t graph_ = nullptr;
  hipGraphExec_t graph_exec_ = nullptr;
};

}  // namespace mrt
