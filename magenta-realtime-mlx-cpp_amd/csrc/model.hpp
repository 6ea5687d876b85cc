// Host orchestration of the Depthformer HIP backend: device weights (Model)
// and one decode stream's device state (State).  Mirrors the reference's
// ``Depthformer`` class (depthformer/model.h:72-239) and ``generate_tokens``
// (depthformer/decode.cpp:239-573).
#pragma once

#include <hip/hip_runtime.h>

#include <memory>
#include <string>
#include <mutex>
#include <vector>

#include "common.hpp"
#include "persist.hpp"
#include "safetensors.hpp"

namespace mrt {

// DepthformerConfig (model.h:47-68).
struct Config {
  int vocab_size = 29824;
  int d_model = 768;
  int d_kv = 64;
  int d_ff = 2048;
  int num_heads = 12;
  int num_encoder_layers = 12;
  int num_temporal_layers = 20;
  int num_depth_layers = 4;
  int max_encoder_length = 1006;
  int rvq_depth = 16;
  int temporal_num_buckets = 128;
  int temporal_max_distance = 128;
  int depth_num_buckets = 16;
  int depth_max_distance = 16;

  static Config base() { return Config{}; }  // model.cpp:34-36
  static Config large() {                     // model.cpp:38-48
    Config c;
    c.d_model = 1024;
    c.d_kv = 64;
    c.d_ff = 2816;
    c.num_heads = 16;
    c.num_encoder_layers = 24;
    c.num_temporal_layers = 40;
    c.num_depth_layers = 8;
    return c;
  }
  int hd() const { return num_heads * d_kv; }
};

// T5 relative-position bucket for a non-negative query-key distance n
// (unidirectional branch of modules.cpp:139-174, float32 log branch).
int relative_position_bucket(int n, int num_buckets, int max_distance);

// Bundle key -> shape for a config (the reference's weight-bundle layout).
std::vector<std::pair<std::string, std::vector<int64_t>>> bundle_layout(const Config& c);

struct EncoderLayerW {
  const void *norm_attn, *wqkv, *wo, *norm_ff, *w01, *wo2;
};
struct DecoderLayerW {
  const void *norm_sa, *wqkv, *wo, *norm_ca, *wq_c, *wo_c, *norm_ff, *w01, *wo2;
};

struct GenOpts;

class Model {
 public:
  Model(const TensorSource& src, const Config& cfg, DType dt, int device);
  ~Model();
  Model(const Model&) = delete;
  Model& operator=(const Model&) = delete;

  Config cfg;
  DType dt;
  int device;
  size_t esz;  // bytes per stored element

  const void* emb = nullptr;       // (V, D)
  const void* lm_head = nullptr;   // (V, D)
  const void* pe = nullptr;        // (max_enc, D), rounded to the model dtype
  const void* enc_norm = nullptr;  // (D)
  const void* dec_norm = nullptr;  // (D)
  const void* tbias = nullptr;     // (temporal buckets, H)
  const void* dbias = nullptr;     // (depth buckets, H)
  const int* tbuckets = nullptr;   // bucket of distance n, n < kBucketTable
  const int* dbuckets = nullptr;
  const void* wkv_cross = nullptr; // (Lt * 2 * HD, D): [layer][k|v] rows
  // Self-attention bias rows of positions 0..kBiasRows-1, model dtype, as
  // precompute_biases lays them out (position p's (H, p + 1) block at element
  // H p (p + 1) / 2): the persistent kernels read one element per key.
  const void* tbias_rows = nullptr;
  const void* dbias_rows = nullptr;
  static constexpr int kBiasRows = 64;
  std::vector<EncoderLayerW> enc;
  std::vector<DecoderLayerW> tmp, dep;
  size_t weight_bytes = 0;

  static constexpr int kBucketTable = 4096;

  // One draw as State::sample without a state and without allocating: the
  // (2, codebook) fp32 device slice in, the LLM id to token_dev[0], enqueued
  // on `stream` (no wait).  Scratch is the library's fixed per-device array.
  void sample_noalloc(const float* slice_dev, const GenOpts& o, int frame, int level, int32_t* token_dev,
                      hipStream_t stream) const;
  // Depthformer::token_embedding()(ids) (model.h:127, modules.cpp:110-112),
  // as the decode loop embeds every fed token (decode.cpp:366-368, 476-477):
  // rows emb[ids[i]] (model dtype) of n host ids into the device buffer
  // `out` (n, d_model), enqueued on `s`; waits for it.
  void embed_tokens(const int32_t* ids, int n, void* out, hipStream_t s);
  // Depthformer::position_embedding(seq_len) (model.cpp:215-224): the first
  // seq_len rows of the fp32 sinusoid table into the device buffer `out`.
  void position_embedding(int seq_len, float* out) const;
  // precompute_{temporal,depth}_biases (model.cpp:302-320): kind 0 temporal,
  // 1 depth; steps 0..n-1 back to back into the device buffer `out` (step f's
  // (H, f + 1) block at element H f (f + 1) / 2).  Waits for the result.
  void precompute_biases(int kind, int n, void* out) const;

  // The first depth layer's q | k | v of every token the decode feeds back at
  // levels 1..rvq_depth-1: row ((l - 1) * codebook + c) is
  // round(Wqkv0 . rmsnorm(emb(offset + codebook * (l - 1) + c))), 3 * HD
  // model-dtype values -- the layer-0 projection of depth step l when its input
  // is that token's embedding on both rows.  Built on first use for a
  // (codebook, offset) pair, on `s` (waits for it; never during a capture), and
  // kept until the model is destroyed: (rvq_depth - 1) * codebook * 3 * HD
  // elements (94 MB in bf16 at d_model 1024, codebook 1024), plus a
  // kQkvChunkRows x d_model build workspace allocated once.  The first build
  // for a pair allocates its table (hipMalloc) and frees nothing.  At most
  // kMaxQkvTables pairs get a table; nullptr for any other pair and when
  // levels < 2 (the decode then computes layer 0).
  const void* depth_qkv_table(int codebook, int offset, hipStream_t s);
  static constexpr size_t kMaxQkvTables = 4;
  static constexpr int kQkvChunkRows = 2048;

 private:
  std::vector<void*> allocs_;
  struct QkvTable {
    int codebook, offset;
    void* rows;
  };
  std::mutex qkv_mu_;
  std::vector<QkvTable> qkv_tables_;
  void* qkv_ws_ = nullptr;  // build workspace of the tables (kQkvChunkRows x d_model)
  std::vector<float> pe_host_;  // fp32 sinusoid table (max_encoder_length, d_model)
  static constexpr int kEmbedChunk = 4096;
  std::mutex embed_mu_;
  int* embed_ids_dev_ = nullptr;       // kEmbedChunk ids, allocated at the first embed_tokens
  int32_t* embed_ids_host_ = nullptr;  // pinned staging of the same
  const void* upload(const std::vector<float>& host);
  const void* upload_i32(const std::vector<int>& host);
};

// Encoder workspace for `rows` rows of S token ids (2 rows per stream).
struct EncoderBufs {
  int rows = 0, S = 0;
  int* tok = nullptr;  // (rows, S) ids, range-checked by whoever wrote them
  void *ex = nullptr, *exn = nullptr, *eqkv = nullptr, *eattn = nullptr, *effh = nullptr;
  void* enc_out = nullptr;  // (rows, S, d_model)
  void* cross = nullptr;    // (Lt, k|v, rows, H, S, 64)
};
// Depthformer::encode (model.cpp:226-241) over every row, then the cross K/V
// of every temporal layer (modules.cpp:448-455).
void run_encoder(const Model& m, const EncoderBufs& b, hipStream_t s);
void project_cross_kv(const Model& m, const void* enc_out, int rows, int S, void* cross, hipStream_t s);

struct GenOpts {
  int num_frames = 50;
  int rvq_depth = 16;
  float temperature = 1.1f;
  int top_k = 40;
  float guidance_weight = 4.0f;
  uint64_t seed = 0;
  int codebook = 1024;
  int codec_offset = 2;
  const int32_t* teacher = nullptr;  // host (F, L)
  bool use_graph = false;
  // Speculative depth decoding (decode.cpp:150-237, 380-446) with the previous
  // call's tokens as the drafts: bf16 persistent path, no teacher.
  bool speculative = false;
  // Speculate only the first spec_frames frames (0: every frame); the rest of
  // the chunk decodes as usual.  The stream's adaptive mode probes with it.
  int spec_frames = 0;
  float* record_slices = nullptr;    // device (F, L, rows, C)
  void* record_temporal = nullptr;   // device (F, rows, D)
  int* record_drawn = nullptr;       // device (F, L)
  void* record_frame_mean = nullptr; // device (F, rows, D)
};

class State {
 public:
  State(Model& m, int rows, int max_frames, int enc_len);
  ~State();
  State(const State&) = delete;
  State& operator=(const State&) = delete;

  Model& m;
  int rows, F, S;
  hipStream_t stream = nullptr;

  void encode(const int32_t* tokens_host);
  void encode_device();  // encoder on the ids in enc_tokens_dev()
  int* enc_tokens_dev() const { return d_enc_tok; }
  int* tokens_dev() const { return d_tokens; }
  void project_cross(const void* enc_out_dev);
  // bias: the reference's optional position_bias, (H, idx + 1) model dtype
  // device rows replacing the rel-pos table lookup, or nullptr.
  void temporal_step(const void* in, const void* enc_out, int frame_idx, void* out, const void* bias = nullptr);
  void depth_step(const void* in, int depth_idx, int level, int codebook, int codec_offset,
                  float* logits, const void* bias = nullptr);
  // Drops the temporal (kind 0) or depth (kind 1) cache contents: the next step
  // of that kind must be at index 0 (empty_{temporal,depth}_cache, model.cpp:275-300).
  void reset_cache(int kind);

  void generate(const int32_t* enc_tokens_host, const GenOpts& o, int32_t* out_host);
  // Full-sequence depth pass over k positions (model.cpp:243-268): emb (2, k, D)
  // model dtype, bias (H, k, k) model dtype or nullptr, logits (2, k, vocab) fp32.
  void depth_forward_full(const void* emb, int k, const void* bias, bool causal, float* logits);
  // CFG + temperature/top-k draw over one level slice (rows 0/1, C entries)
  // held in a device fp32 buffer; returns the LLM id.
  int sample(const float* slice_dev, const GenOpts& o, int frame, int level);

  // Buffer access for parity checks.
  void* buffer(int which, int layer, size_t* bytes);
  void set_cache_length(int kind, int length);
  void sync();
  bool persistent() const { return persist_grid_ > 0; }
  // GPU ms of the decode section (after the encoder) of the last generate
  // call, from HIP events on the state's stream; launches = persistent
  // kernel launches in it (0 on the per-layer path).
  // Share of the last generate's levels whose token came from the verification
  // pass (accepted drafts and the first disagreement); -1 when it did not speculate.
  float spec_acceptance() const { return spec_acc_; }
  float last_decode_ms(int* launches);
  // Depthformer::compile_for_inference (model.cpp:709-...): prepares this
  // state's decode for options `o` ahead of the first real call -- the layer-0
  // q/k/v table, the captured decode graph (o.use_graph) and the first launch of
  // every kernel on the path -- by one untimed decode (two when o.speculative,
  // so the speculative graph is captured too) on the current encoder output, or
  // on an encoding of PAD ids when there is none.  Afterwards the caches and the
  // draft history are as before (no encoder output stays if there was none).
  void compile(const GenOpts& o);
  // Per-phase GPU times of the last generate call (the MRT_PROFILE_DECODE
  // breakdown of decode.cpp:36-49, 529-565).  The temporal / depth / draw split
  // comes from workgroup 0's wall-clock stamps inside the frame kernel, taken
  // while profiling is on (MRT_PROFILE_DECODE set when the state was created,
  // or set_profile); -1 where the last call did not record it.
  struct DecodeProfile {
    float total_ms = -1.f, encoder_ms = -1.f, temporal_ms = -1.f, depth_ms = -1.f, sample_ms = -1.f;
    int frames = 0;
  };
  void set_profile(bool on) { profile_ = on; }
  DecodeProfile decode_profile();
  // Raw per-phase timeline of workgroup 0 (MRT_TRACE_PHASES set at state
  // creation): 2 x kTraceSlots device wall-clock stamps, the temporal step and
  // depth level 1 of frame 1 of the last decode.  Returns the clock in MHz.
  float phase_trace(uint64_t* out, int n);

 private:
  // Persistent-kernel decode path: one launch per step (API steps) or per
  // frame (decode loop).
  void setup_persistent();
  StepArgs temporal_args(const void* in, int f, void* out) const;
  StepArgs depth_args(const void* in, int l, const void* head_w, int head_rows, float* logits,
                      float* rec_slice) const;
  void launch_temporal_p(const void* in, int f, void* out, const void* bias = nullptr);
  void launch_depth_p(const void* in, int l, const void* head_w, int head_rows, float* logits, float* rec_slice,
                      const void* bias = nullptr);
  void launch_frame_p(const GenOpts& o, int f);
  void enqueue_decode_p(const GenOpts& o);
  void enqueue_decode_spec(const GenOpts& o);
  bool speculating(const GenOpts& o) const;
  int spec_count(const GenOpts& o) const;  // frames of this call that speculate
  void enqueue_plain_frame(const GenOpts& o, int f, const SampleParams& sp);
  int decode_launches(const GenOpts& o) const;
  void reserve_epochs(uint32_t n);
  void check_device_error();
  int persist_grid_ = 0, bph_ = 0;
  bool frame_kernel_ = false;  // the decode loop runs one launch per frame
  void* ll_block_ = nullptr;
  size_t ll_words_ = 0;
  uint32_t epochs_used_ = 0;   // launches since the hand-off words were zeroed
  LLBufs ll_bufs(int stack = 1) const;  // hand-off words; delays of stack 0 (temporal) or 1 (depth)
  void reset_handoff();
  DecStack tstack_{}, dstack_{};  // temporal / depth stacks with this state's caches
  size_t lds_t_ = 0, lds_d_ = 0, lds_f_ = 0, lds_l_ = 0;  // dynamic LDS of the persistent kernels
  float* noise_ = nullptr;         // Gumbel noise of every draw of a decode call
  int* h_err_ = nullptr;        // pinned
  uint64_t* h_seed_ = nullptr;  // pinned: the draw seed of a generate / sample call
  uint64_t* d_trace_ = nullptr; // 2 x kTraceSlots when MRT_TRACE_PHASES is set
  uint8_t poll_delay_[2][kPollSites];  // per stack (temporal, depth) and poll site: s_sleep(1) rounds before a hand-off's first poll
  bool qkv_table_on_ = true;    // frame kernel: layer-0 q/k/v of fed tokens from the model's table (MRT_QKV_TABLE=0: off)
  const void* qkv_table_ = nullptr;  // the table of the current generate call, or nullptr
  hipEvent_t ev_dec_[2] = {nullptr, nullptr};  // around the decode section of generate
  hipEvent_t ev_enc_[2] = {nullptr, nullptr};  // around the last encoder pass
  bool enc_timed_ = false;
  bool profile_ = false;           // frame kernel phase stamps (MRT_PROFILE_DECODE)
  uint64_t* d_prof_ = nullptr;     // (F, 4) stamps of the last decode
  uint64_t* h_prof_ = nullptr;     // pinned copy
  int prof_frames_ = 0;            // frames stamped by the last decode (0: none)
  int dec_launches_ = 0;
  bool dec_timed_ = false;
  // speculative decoding: drafts (the previous call's tokens), the
  // verification pass's rows (2 L) and its per-level draws / accepted count
  int* d_drafts_ = nullptr;
  int prev_frames_ = 0;  // frames of the tokens left by the last generate (0: none)
  bool spec_drafts_ = false;  // this call speculates with d_drafts_
  void *sx_ = nullptr, *sxn_ = nullptr, *sq_ = nullptr, *satt_ = nullptr, *sffh_ = nullptr, *sqkv_ = nullptr;
  float* slog_ = nullptr;
  int *sdrawn_ = nullptr, *sdecided_ = nullptr;  // sdecided_: (F) the accepted count n of each frame
  float spec_acc_ = -1.f;  // share of the last call's levels taken from the verification pass
  void* sfm_ = nullptr;  // scratch frame-mean rows of the sampler (the spec path writes its own)
  void print_trace();

  size_t esz() const { return m.esz; }
  char* tk(int i) const;
  char* tv(int i) const;
  char* dk(int i) const;
  char* dv(int i) const;
  char* ck(int i) const;
  char* cv(int i) const;
  void run_temporal(const void* in, int f, void* out, const void* bias = nullptr);
  void run_depth(const void* in, int l, int level, int codebook, int codec_offset, float* logits,
                 const void* bias = nullptr);
  void enqueue_decode(const GenOpts& o);
  void copy(void* dst, const void* src, size_t bytes);

  std::vector<void*> allocs_;
  void* dalloc(size_t bytes);

  // device buffers
  int* d_enc_tok = nullptr;
  int32_t* h_pinned = nullptr;  // host staging: tokens in/out
  size_t h_pinned_n = 0;
  void *ex = nullptr, *exn = nullptr, *eqkv = nullptr, *eattn = nullptr, *effh = nullptr;
  void* enc_out = nullptr;
  void *cross = nullptr, *tkv = nullptr, *dkv = nullptr;
  void *x = nullptr, *q = nullptr, *attn = nullptr, *ffh = nullptr;
  void *t_in = nullptr, *t_out = nullptr, *d_in = nullptr, *fsum = nullptr;
  float *slice = nullptr, *part = nullptr;
  int *d_tokens = nullptr, *d_teacher = nullptr;
  uint64_t* d_seed = nullptr;
  int nsplit = 1;
  int max_slice = 0;

  int temporal_len_ = 0, depth_len_ = 0;
  bool cross_ready_ = false;

  // captured decode loops, one per option key (plain and speculative chunks
  // of adaptive streaming alternate without re-capturing); least recently
  // used evicted beyond kMaxDecodeGraphs
  struct DecodeGraph {
    std::vector<double> key;
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    uint64_t used = 0;
  };
  static constexpr size_t kMaxDecodeGraphs = 4;
  std::vector<DecodeGraph> graphs_;
  uint64_t graph_clock_ = 0;
  hipGraphExec_t decode_graph(const GenOpts& o);
  void enqueue_decode_any(const GenOpts& o);
};

}  // namespace mrt
