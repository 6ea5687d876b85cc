// extern "C" boundary of the Depthformer HIP backend (include/mrt_df.h).
// Every entry point converts C++ exceptions into a status code and a
// thread-local message; nothing throws across the ABI.
#include "../../include/mrt_df.h"

#include <memory>
#include <string>

#include "batch.hpp"
#include "coca.hpp"
#include "codec.hpp"
#include "model.hpp"
#include "stream.hpp"

struct mrt_df {
  std::unique_ptr<mrt::Model> model;
};

struct mrt_df_state {
  mrt_df* owner = nullptr;
  std::unique_ptr<mrt::State> owned;
  mrt::State* state = nullptr;  // owned.get(), or a stream's state
};

struct mrt_df_batch {
  std::unique_ptr<mrt::Batch> batch;
};

struct mrt_codec {
  std::unique_ptr<mrt::Codec> codec;
};

struct mrt_coca {
  std::unique_ptr<mrt::Coca> coca;
};

struct mrt_df_stream {
  mrt_df* owner = nullptr;
  std::unique_ptr<mrt::Stream> stream;
  mrt_df_state view;  // borrowed handle on stream->st
};

namespace {

thread_local std::string g_last_error;

template <class Fn>
int guarded(Fn&& fn) {
  try {
    g_last_error.clear();
    fn();
    return MRT_OK;
  } catch (const mrt::Error& e) {
    g_last_error = e.what();
    return e.code;
  } catch (const std::exception& e) {
    g_last_error = e.what();
    return MRT_ERR_INTERNAL;
  } catch (...) {
    g_last_error = "unknown error";
    return MRT_ERR_INTERNAL;
  }
}

mrt::Config to_config(const mrt_df_config* c) {
  mrt::Config k;
  k.vocab_size = c->vocab_size;
  k.d_model = c->d_model;
  k.d_kv = c->d_kv;
  k.d_ff = c->d_ff;
  k.num_heads = c->num_heads;
  k.num_encoder_layers = c->num_encoder_layers;
  k.num_temporal_layers = c->num_temporal_layers;
  k.num_depth_layers = c->num_depth_layers;
  k.max_encoder_length = c->max_encoder_length;
  k.rvq_depth = c->rvq_depth;
  k.temporal_num_buckets = c->temporal_num_buckets;
  k.temporal_max_distance = c->temporal_max_distance;
  k.depth_num_buckets = c->depth_num_buckets;
  k.depth_max_distance = c->depth_max_distance;
  return k;
}

void from_config(const mrt::Config& k, mrt_df_config* c) {
  c->vocab_size = k.vocab_size;
  c->d_model = k.d_model;
  c->d_kv = k.d_kv;
  c->d_ff = k.d_ff;
  c->num_heads = k.num_heads;
  c->num_encoder_layers = k.num_encoder_layers;
  c->num_temporal_layers = k.num_temporal_layers;
  c->num_depth_layers = k.num_depth_layers;
  c->max_encoder_length = k.max_encoder_length;
  c->rvq_depth = k.rvq_depth;
  c->temporal_num_buckets = k.temporal_num_buckets;
  c->temporal_max_distance = k.temporal_max_distance;
  c->depth_num_buckets = k.depth_num_buckets;
  c->depth_max_distance = k.depth_max_distance;
}

mrt::DType to_dtype(int d) {
  if (d == MRT_DTYPE_F32) return mrt::DType::F32;
  if (d == MRT_DTYPE_BF16) return mrt::DType::BF16;
  if (d == MRT_DTYPE_F16) return mrt::DType::F16;
  throw mrt::Error(MRT_ERR_INVALID, "unknown dtype " + std::to_string(d) + "; expected fp32|fp16|bf16");
}

mrt::GenOpts to_opts(const mrt_gen_opts* opts) {
  mrt::GenOpts o;
  o.num_frames = opts->num_frames;
  o.rvq_depth = opts->rvq_depth;
  o.temperature = opts->temperature;
  o.top_k = opts->top_k;
  o.guidance_weight = opts->guidance_weight;
  o.seed = opts->seed;
  o.codebook = opts->codebook_size;
  o.codec_offset = opts->codec_offset;
  o.teacher = opts->teacher;
  o.use_graph = opts->use_graph != 0;
  o.record_slices = opts->record_slices;
  o.record_temporal = opts->record_temporal;
  o.record_drawn = opts->record_drawn;
  o.record_frame_mean = opts->record_frame_mean;
  o.speculative = opts->speculative != 0;
  return o;
}

mrt::State& S(mrt_df_state* st) {
  if (!st || !st->state) throw mrt::Error(MRT_ERR_INVALID, "null state handle");
  return *st->state;
}

mrt::Batch& BB(mrt_df_batch* b) {
  if (!b || !b->batch) throw mrt::Error(MRT_ERR_INVALID, "null batch handle");
  return *b->batch;
}

mrt::Stream& SS(mrt_df_stream* s) {
  if (!s || !s->stream) throw mrt::Error(MRT_ERR_INVALID, "null stream handle");
  return *s->stream;
}

mrt::Coca& CO(mrt_coca* h) {
  if (!h || !h->coca) throw mrt::Error(MRT_ERR_INVALID, "null style-model handle");
  return *h->coca;
}

mrt::CocaConfig to_coca_config(const mrt_coca_config* c) {
  mrt::CocaConfig k;
  k.d_model = c->d_model;
  k.num_heads = c->num_heads;
  k.d_head = c->d_head;
  k.d_ff = c->d_ff;
  k.num_layers = c->num_layers;
  k.pooler_d_head = c->pooler_d_head;
  k.vocab_size = c->vocab_size;
  k.max_text_len = c->max_text_len;
  k.rvq_depth = c->rvq_depth;
  k.codebook = c->codebook_size;
  if (k.num_layers < 1 || k.num_heads < 1 || k.vocab_size < 1)
    throw mrt::Error(MRT_ERR_INVALID, "musiccoca: layers, heads and vocabulary must be >= 1");
  return k;
}

mrt::Codec& CC(mrt_codec* c) {
  if (!c || !c->codec) throw mrt::Error(MRT_ERR_INVALID, "null codec handle");
  return *c->codec;
}

mrt::CodecConfig to_codec_config(const mrt_codec_config* c, int* max_frames) {
  mrt::CodecConfig k;
  k.embedding_dim = c->embedding_dim;
  k.proj_ch = c->proj_channels;
  k.unfold = c->unfold;
  for (int i = 0; i < 7; ++i) {
    k.blocks[i].in_ch = c->block_in[i];
    k.blocks[i].out_ch = c->block_out[i];
  }
  k.levels = c->rvq_levels;
  k.codebook = c->codebook_size;
  if (k.levels < 1 || k.codebook < 1) throw mrt::Error(MRT_ERR_INVALID, "codec: rvq_levels and codebook_size must be >= 1");
  *max_frames = c->max_frames;
  return k;
}

mrt::ChunkOpts to_chunk_opts(const mrt_chunk_opts* opts) {
  mrt::ChunkOpts o;
  o.temperature = opts->temperature;
  o.top_k = opts->top_k;
  o.guidance_weight = opts->guidance_weight;
  o.has_seed = opts->has_seed != 0;
  o.seed = opts->seed;
  o.pipeline_encoder = opts->pipeline_encoder != 0;
  o.use_graph = opts->use_graph != 0;
  o.teacher = opts->teacher;
  o.speculative = opts->speculative;
  return o;
}

mrt::StreamConfig to_stream_config(const mrt_stream_config* c) {
  mrt::StreamConfig k;
  k.chunk_frames = c->chunk_frames;
  k.context_frames = c->context_frames;
  k.codebook = c->codebook_size;
  k.enc_depth = c->encoder_codec_rvq_depth;
  k.style_depth = c->encoder_style_rvq_depth;
  k.levels = c->decoder_codec_rvq_depth;
  k.mask = c->mask_token;
  k.codec_offset = c->codec_offset;
  k.crossfade_frames = c->crossfade_frames;
  k.samples_per_frame = c->samples_per_frame;
  return k;
}

}  // namespace

extern "C" {

const char* mrt_last_error(void) { return g_last_error.c_str(); }

void mrt_df_config_base(mrt_df_config* cfg) {
  if (cfg) from_config(mrt::Config::base(), cfg);
}

void mrt_df_config_large(mrt_df_config* cfg) {
  if (cfg) from_config(mrt::Config::large(), cfg);
}

int mrt_df_create(const char* bundle_path, const mrt_df_config* cfg, int dtype, int device, mrt_df** out) {
  return guarded([&] {
    if (!bundle_path || !cfg || !out) throw mrt::Error(MRT_ERR_INVALID, "null argument");
    *out = nullptr;
    mrt::SafetensorsFile src(bundle_path);
    auto h = std::make_unique<mrt_df>();
    h->model = std::make_unique<mrt::Model>(src, to_config(cfg), to_dtype(dtype), device);
    *out = h.release();
  });
}

int mrt_df_create_from_tensors(int n, const char* const* names, const float* const* data,
                               const int64_t* const* shapes, const int32_t* ndims, const mrt_df_config* cfg,
                               int dtype, int device, mrt_df** out) {
  return guarded([&] {
    if (!names || !data || !shapes || !ndims || !cfg || !out || n < 0)
      throw mrt::Error(MRT_ERR_INVALID, "null argument");
    *out = nullptr;
    mrt::TensorList src;
    for (int i = 0; i < n; ++i) {
      if (!names[i] || !data[i] || ndims[i] < 0) throw mrt::Error(MRT_ERR_INVALID, "bad tensor entry");
      src.add(names[i], data[i], std::vector<int64_t>(shapes[i], shapes[i] + ndims[i]));
    }
    auto h = std::make_unique<mrt_df>();
    h->model = std::make_unique<mrt::Model>(src, to_config(cfg), to_dtype(dtype), device);
    *out = h.release();
  });
}

void mrt_df_destroy(mrt_df* h) { delete h; }

int mrt_df_get_config(const mrt_df* h, mrt_df_config* cfg, int* dtype) {
  return guarded([&] {
    if (!h || !h->model) throw mrt::Error(MRT_ERR_INVALID, "null model handle");
    if (cfg) from_config(h->model->cfg, cfg);
    if (dtype) *dtype = static_cast<int>(h->model->dt);
  });
}

int mrt_df_state_create(mrt_df* h, int rows, int max_frames, int enc_len, mrt_df_state** out) {
  return guarded([&] {
    if (!h || !h->model || !out) throw mrt::Error(MRT_ERR_INVALID, "null argument");
    *out = nullptr;
    auto st = std::make_unique<mrt_df_state>();
    st->owner = h;
    st->owned = std::make_unique<mrt::State>(*h->model, rows, max_frames, enc_len);
    st->state = st->owned.get();
    *out = st.release();
  });
}

void mrt_df_state_destroy(mrt_df_state* st) {
  if (st && st->owned) delete st;  // a stream's borrowed handle is freed with the stream
}

int mrt_df_state_stream(mrt_df_state* st, void** hip_stream) {
  return guarded([&] {
    if (!hip_stream) throw mrt::Error(MRT_ERR_INVALID, "null argument");
    *hip_stream = S(st).stream;
  });
}

int mrt_df_sync(mrt_df_state* st) {
  return guarded([&] { S(st).sync(); });
}

int mrt_df_encode(mrt_df_state* st, const int32_t* tokens) {
  return guarded([&] {
    if (!tokens) throw mrt::Error(MRT_ERR_INVALID, "null tokens");
    S(st).encode(tokens);
  });
}

int mrt_df_temporal_step(mrt_df_state* st, const void* frame_emb, const void* enc_out, int frame_idx,
                         void* out) {
  return guarded([&] {
    if (!frame_emb || !out) throw mrt::Error(MRT_ERR_INVALID, "null argument");
    S(st).temporal_step(frame_emb, enc_out, frame_idx, out);
  });
}

int mrt_df_depth_step(mrt_df_state* st, const void* tok_emb, int depth_idx, int level, int codebook_size,
                      int codec_offset, float* logits) {
  return guarded([&] {
    if (!tok_emb || !logits) throw mrt::Error(MRT_ERR_INVALID, "null argument");
    S(st).depth_step(tok_emb, depth_idx, level, codebook_size, codec_offset, logits);
  });
}

int mrt_df_temporal_step_with_bias(mrt_df_state* st, const void* frame_emb, const void* enc_out, int frame_idx,
                                   const void* position_bias, void* out) {
  return guarded([&] {
    if (!frame_emb || !out || !position_bias) throw mrt::Error(MRT_ERR_INVALID, "null argument");
    S(st).temporal_step(frame_emb, enc_out, frame_idx, out, position_bias);
  });
}

int mrt_df_depth_step_with_bias(mrt_df_state* st, const void* tok_emb, int depth_idx, const void* position_bias,
                                int level, int codebook_size, int codec_offset, float* logits) {
  return guarded([&] {
    if (!tok_emb || !logits || !position_bias) throw mrt::Error(MRT_ERR_INVALID, "null argument");
    S(st).depth_step(tok_emb, depth_idx, level, codebook_size, codec_offset, logits, position_bias);
  });
}

int mrt_df_precompute_biases(mrt_df* h, int kind, int n, void* out) {
  return guarded([&] {
    if (!h || !out) throw mrt::Error(MRT_ERR_INVALID, "null argument");
    h->model->precompute_biases(kind, n, out);
  });
}

int mrt_df_state_reset_cache(mrt_df_state* st, int kind) {
  return guarded([&] { S(st).reset_cache(kind); });
}

int mrt_df_generate_tokens(mrt_df_state* st, const int32_t* enc_tokens, const mrt_gen_opts* opts,
                           int32_t* out_tokens) {
  return guarded([&] {
    if (!opts || !out_tokens) throw mrt::Error(MRT_ERR_INVALID, "null argument");
    S(st).generate(enc_tokens, to_opts(opts), out_tokens);
  });
}

int mrt_df_sample_level(mrt_df_state* st, const float* slice, const mrt_gen_opts* opts, int frame, int level,
                        int32_t* token) {
  return guarded([&] {
    if (!slice || !opts || !token) throw mrt::Error(MRT_ERR_INVALID, "null argument");
    *token = S(st).sample(slice, to_opts(opts), frame, level);
  });
}

int mrt_df_depth_forward_full(mrt_df_state* st, const void* token_embeddings, int k_len, const void* position_bias,
                              int causal, float* logits) {
  return guarded([&] {
    if (!token_embeddings || !logits) throw mrt::Error(MRT_ERR_INVALID, "null argument");
    S(st).depth_forward_full(token_embeddings, k_len, position_bias, causal != 0, logits);
  });
}

int mrt_df_sample_level_noalloc(mrt_df* h, const float* slice_dev, const mrt_gen_opts* opts, int frame, int level,
                                int32_t* token_dev, void* hip_stream) {
  return guarded([&] {
    if (!h || !slice_dev || !opts || !token_dev) throw mrt::Error(MRT_ERR_INVALID, "null argument");
    h->model->sample_noalloc(slice_dev, to_opts(opts), frame, level, token_dev,
                             static_cast<hipStream_t>(hip_stream));
  });
}

int mrt_df_state_decode_time(mrt_df_state* st, float* ms, int* launches) {
  return guarded([&] {
    if (!ms) throw mrt::Error(MRT_ERR_INVALID, "null argument");
    *ms = S(st).last_decode_ms(launches);
  });
}

int mrt_df_state_phase_trace(mrt_df_state* st, uint64_t* out, int n, float* clock_mhz) {
  return guarded([&] {
    if (!out || !clock_mhz) throw mrt::Error(MRT_ERR_INVALID, "null argument");
    *clock_mhz = S(st).phase_trace(out, n);
  });
}

int mrt_df_state_set_profile(mrt_df_state* st, int on) {
  return guarded([&] { S(st).set_profile(on != 0); });
}

int mrt_df_state_decode_profile(mrt_df_state* st, mrt_decode_profile* out) {
  return guarded([&] {
    if (!out) throw mrt::Error(MRT_ERR_INVALID, "null argument");
    const mrt::State::DecodeProfile p = S(st).decode_profile();
    out->total_ms = p.total_ms;
    out->encoder_ms = p.encoder_ms;
    out->bias_ms = 0.f;
    out->temporal_ms = p.temporal_ms;
    out->depth_ms = p.depth_ms;
    out->sample_ms = p.sample_ms;
    out->frames = p.frames;
  });
}

int mrt_df_state_compile(mrt_df_state* st, const mrt_gen_opts* opts) {
  return guarded([&] {
    if (!opts) throw mrt::Error(MRT_ERR_INVALID, "null argument");
    S(st).compile(to_opts(opts));
  });
}

int mrt_df_embed_tokens(mrt_df* h, const int32_t* ids, int n, void* out, void* hip_stream) {
  return guarded([&] {
    if (!h || !h->model || (n > 0 && (!ids || !out))) throw mrt::Error(MRT_ERR_INVALID, "null argument");
    h->model->embed_tokens(ids, n, out, static_cast<hipStream_t>(hip_stream));
  });
}

int mrt_df_position_embedding(mrt_df* h, int seq_len, float* out) {
  return guarded([&] {
    if (!h || !h->model || (seq_len > 0 && !out)) throw mrt::Error(MRT_ERR_INVALID, "null argument");
    h->model->position_embedding(seq_len, out);
  });
}

int mrt_df_state_spec_acceptance(mrt_df_state* st, float* acceptance) {
  return guarded([&] {
    if (!acceptance) throw mrt::Error(MRT_ERR_INVALID, "null argument");
    *acceptance = S(st).spec_acceptance();
  });
}

int mrt_probe_read_bandwidth(int device, size_t bytes, int passes, float* gbps) {
  return guarded([&] {
    if (!gbps) throw mrt::Error(MRT_ERR_INVALID, "null argument");
    *gbps = mrt::probe_read_bandwidth(device, bytes, passes);
  });
}

int mrt_probe_handoff(int device, int workgroups, int words, int rounds, int delay, float* us_per_round) {
  return guarded([&] {
    if (!us_per_round) throw mrt::Error(MRT_ERR_INVALID, "null argument");
    *us_per_round = mrt::probe_handoff(device, workgroups, words, rounds, delay);
  });
}

int mrt_probe_pingpong(int device, int peer, int rounds, float* us_one_way) {
  return guarded([&] {
    if (!us_one_way) throw mrt::Error(MRT_ERR_INVALID, "null argument");
    *us_one_way = mrt::probe_pingpong(device, peer, rounds);
  });
}

int mrt_df_state_buffer_bytes(mrt_df_state* st, int which, size_t* bytes) {
  return guarded([&] {
    if (!bytes) throw mrt::Error(MRT_ERR_INVALID, "null argument");
    S(st).buffer(which, 0, bytes);
  });
}

int mrt_df_state_read(mrt_df_state* st, int which, int layer, void* dst, size_t bytes) {
  return guarded([&] {
    if (!dst) throw mrt::Error(MRT_ERR_INVALID, "null argument");
    size_t n = 0;
    void* src = S(st).buffer(which, layer, &n);
    if (bytes != n) throw mrt::Error(MRT_ERR_INVALID, "state_read: size mismatch (" + std::to_string(n) + " bytes)");
    MRT_HIP_CHECK(hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToDevice, S(st).stream));
    S(st).sync();
  });
}

int mrt_df_state_write(mrt_df_state* st, int which, int layer, const void* src, size_t bytes) {
  return guarded([&] {
    if (!src) throw mrt::Error(MRT_ERR_INVALID, "null argument");
    size_t n = 0;
    void* dst = S(st).buffer(which, layer, &n);
    if (which == MRT_BUF_ENC_TOKENS) throw mrt::Error(MRT_ERR_INVALID, "state_write: the encoder ids are read-only");
    if (bytes != n) throw mrt::Error(MRT_ERR_INVALID, "state_write: size mismatch (" + std::to_string(n) + " bytes)");
    MRT_HIP_CHECK(hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToDevice, S(st).stream));
    S(st).sync();
    if (which == MRT_BUF_CROSS_K || which == MRT_BUF_CROSS_V) S(st).set_cache_length(2, 1);
  });
}

int mrt_df_state_set_cache_length(mrt_df_state* st, int kind, int length) {
  return guarded([&] { S(st).set_cache_length(kind, length); });
}

void mrt_stream_config_default(mrt_stream_config* cfg) {
  if (!cfg) return;
  const mrt::StreamConfig k;
  cfg->chunk_frames = k.chunk_frames;
  cfg->context_frames = k.context_frames;
  cfg->codebook_size = k.codebook;
  cfg->encoder_codec_rvq_depth = k.enc_depth;
  cfg->encoder_style_rvq_depth = k.style_depth;
  cfg->decoder_codec_rvq_depth = k.levels;
  cfg->mask_token = k.mask;
  cfg->codec_offset = k.codec_offset;
  cfg->crossfade_frames = k.crossfade_frames;
  cfg->samples_per_frame = k.samples_per_frame;
}

void mrt_chunk_opts_default(mrt_chunk_opts* opts) {
  if (!opts) return;
  const mrt::ChunkOpts k;
  opts->temperature = k.temperature;
  opts->top_k = k.top_k;
  opts->guidance_weight = k.guidance_weight;
  opts->has_seed = 0;
  opts->seed = 0;
  opts->pipeline_encoder = 0;
  opts->use_graph = 1;
  opts->teacher = nullptr;
  opts->speculative = 0;
}

int mrt_df_stream_create(mrt_df* h, const mrt_stream_config* cfg, mrt_df_stream** out) {
  return guarded([&] {
    if (!h || !h->model || !cfg || !out) throw mrt::Error(MRT_ERR_INVALID, "null argument");
    *out = nullptr;
    auto s = std::make_unique<mrt_df_stream>();
    s->owner = h;
    s->stream = std::make_unique<mrt::Stream>(*h->model, to_stream_config(cfg));
    s->view.owner = h;
    s->view.state = &s->stream->st;
    *out = s.release();
  });
}

void mrt_df_stream_destroy(mrt_df_stream* s) { delete s; }

int mrt_df_stream_generate_chunk(mrt_df_stream* s, const int32_t* style, const mrt_chunk_opts* opts,
                                 int32_t* llm_out, int32_t* rvq_out) {
  return guarded([&] {
    if (!opts) throw mrt::Error(MRT_ERR_INVALID, "null argument");
    SS(s).generate_chunk(style, to_chunk_opts(opts), llm_out, rvq_out);
  });
}

int mrt_df_stream_generate_chunk_audio(mrt_df_stream* s, const int32_t* style, const mrt_chunk_opts* opts,
                                       int32_t* llm_out, int32_t* rvq_out, float* audio_out) {
  return guarded([&] {
    if (!opts || !audio_out) throw mrt::Error(MRT_ERR_INVALID, "null argument");
    SS(s).generate_chunk_audio(style, to_chunk_opts(opts), llm_out, rvq_out, audio_out);
  });
}

int mrt_df_stream_compile(mrt_df_stream* s, const mrt_chunk_opts* opts) {
  return guarded([&] {
    if (!opts) throw mrt::Error(MRT_ERR_INVALID, "null argument");
    SS(s).compile(to_chunk_opts(opts));
  });
}

int mrt_df_stream_attach_codec(mrt_df_stream* s, mrt_codec* c) {
  return guarded([&] { SS(s).attach_codec(c ? &CC(c) : nullptr); });
}

int mrt_df_stream_set_context(mrt_df_stream* s, const int32_t* context, int64_t chunk_index) {
  return guarded([&] {
    if (!context) throw mrt::Error(MRT_ERR_INVALID, "null argument");
    SS(s).set_context(context, chunk_index);
  });
}

int mrt_df_stream_get_context(mrt_df_stream* s, int32_t* context, int64_t* chunk_index) {
  return guarded([&] { SS(s).get_context(context, chunk_index); });
}

int mrt_df_stream_state(mrt_df_stream* s, mrt_df_state** st) {
  return guarded([&] {
    if (!st) throw mrt::Error(MRT_ERR_INVALID, "null argument");
    SS(s);
    *st = &s->view;
  });
}

int mrt_df_batch_create(mrt_df* h, int streams, int max_frames, int enc_len, mrt_df_batch** out) {
  return guarded([&] {
    if (!h || !h->model || !out) throw mrt::Error(MRT_ERR_INVALID, "null argument");
    *out = nullptr;
    auto b = std::make_unique<mrt_df_batch>();
    b->batch = std::make_unique<mrt::Batch>(*h->model, streams, max_frames, enc_len);
    *out = b.release();
  });
}

void mrt_df_batch_destroy(mrt_df_batch* b) { delete b; }

int mrt_df_batch_encode(mrt_df_batch* b, const int32_t* tokens) {
  return guarded([&] {
    if (!tokens) throw mrt::Error(MRT_ERR_INVALID, "null tokens");
    BB(b).encode(tokens);
  });
}

int mrt_df_batch_generate_tokens(mrt_df_batch* b, const int32_t* enc_tokens, const mrt_gen_opts* opts,
                                 const uint64_t* seeds, int32_t* out_tokens) {
  return guarded([&] {
    if (!opts || !seeds || !out_tokens) throw mrt::Error(MRT_ERR_INVALID, "null argument");
    if (opts->record_drawn || opts->record_frame_mean)
      throw mrt::Error(MRT_ERR_INVALID, "batch generate: record_drawn / record_frame_mean are not supported");
    BB(b).generate(enc_tokens, to_opts(opts), seeds, out_tokens);
  });
}

int mrt_df_batch_stream(mrt_df_batch* b, void** hip_stream) {
  return guarded([&] {
    if (!hip_stream) throw mrt::Error(MRT_ERR_INVALID, "null argument");
    *hip_stream = BB(b).stream;
  });
}

int mrt_df_batch_decode_time(mrt_df_batch* b, float* ms) {
  return guarded([&] {
    if (!ms) throw mrt::Error(MRT_ERR_INVALID, "null argument");
    *ms = BB(b).last_decode_ms();
  });
}

int mrt_df_batch_read_enc_out(mrt_df_batch* b, void* dst, size_t bytes) {
  return guarded([&] {
    if (!dst) throw mrt::Error(MRT_ERR_INVALID, "null argument");
    mrt::Batch& bt = BB(b);
    const size_t n = static_cast<size_t>(bt.R) * bt.S * bt.m.cfg.d_model * 2;
    if (bytes != n) throw mrt::Error(MRT_ERR_INVALID, "batch_read_enc_out: size mismatch (" + std::to_string(n) + " bytes)");
    MRT_HIP_CHECK(hipMemcpyAsync(dst, bt.enc_out(), n, hipMemcpyDeviceToDevice, bt.stream));
    MRT_HIP_CHECK(hipStreamSynchronize(bt.stream));
  });
}

void mrt_codec_config_default(mrt_codec_config* cfg) {
  if (!cfg) return;
  const mrt::CodecConfig k;
  cfg->embedding_dim = k.embedding_dim;
  cfg->proj_channels = k.proj_ch;
  cfg->unfold = k.unfold;
  for (int i = 0; i < 7; ++i) {
    cfg->block_in[i] = k.blocks[i].in_ch;
    cfg->block_out[i] = k.blocks[i].out_ch;
  }
  cfg->rvq_levels = k.levels;
  cfg->codebook_size = k.codebook;
  cfg->max_frames = 51;
}

int mrt_codec_create(const char* decoder_path, const char* codebooks_path, const mrt_codec_config* cfg, int device,
                     mrt_codec** out) {
  return guarded([&] {
    if (!decoder_path || !codebooks_path || !cfg || !out) throw mrt::Error(MRT_ERR_INVALID, "null argument");
    *out = nullptr;
    int maxf = 0;
    const mrt::CodecConfig k = to_codec_config(cfg, &maxf);
    mrt::SafetensorsFile dec(decoder_path), cbs(codebooks_path);
    auto h = std::make_unique<mrt_codec>();
    h->codec = std::make_unique<mrt::Codec>(dec, cbs, k, device, maxf);
    *out = h.release();
  });
}

int mrt_codec_create_from_tensors(int n, const char* const* names, const float* const* data,
                                  const int64_t* const* shapes, const int32_t* ndims, const mrt_codec_config* cfg,
                                  int device, mrt_codec** out) {
  return guarded([&] {
    if (!names || !data || !shapes || !ndims || !cfg || !out || n < 0)
      throw mrt::Error(MRT_ERR_INVALID, "null argument");
    *out = nullptr;
    int maxf = 0;
    const mrt::CodecConfig k = to_codec_config(cfg, &maxf);
    mrt::TensorList src;
    for (int i = 0; i < n; ++i) {
      if (!names[i] || !data[i] || ndims[i] < 0) throw mrt::Error(MRT_ERR_INVALID, "bad tensor entry");
      src.add(names[i], data[i], std::vector<int64_t>(shapes[i], shapes[i] + ndims[i]));
    }
    auto h = std::make_unique<mrt_codec>();
    h->codec = std::make_unique<mrt::Codec>(src, src, k, device, maxf);
    *out = h.release();
  });
}

void mrt_codec_destroy(mrt_codec* c) { delete c; }

int mrt_codec_decode(mrt_codec* c, const int32_t* rvq_tokens, int frames, float* audio) {
  return guarded([&] { CC(c).decode(rvq_tokens, frames, audio); });
}

int mrt_codec_decode_device(mrt_codec* c, const int32_t* rvq_tokens_dev, int frames, float* audio_dev) {
  return guarded([&] { CC(c).decode_device(rvq_tokens_dev, frames, audio_dev); });
}

int mrt_codec_stream(mrt_codec* c, void** hip_stream) {
  return guarded([&] {
    if (!hip_stream) throw mrt::Error(MRT_ERR_INVALID, "null argument");
    *hip_stream = CC(c).stream;
  });
}

int mrt_codec_sync(mrt_codec* c) {
  return guarded([&] { MRT_HIP_CHECK(hipStreamSynchronize(CC(c).stream)); });
}

int mrt_codec_decode_time(mrt_codec* c, float* ms) {
  return guarded([&] {
    if (!ms) throw mrt::Error(MRT_ERR_INVALID, "null argument");
    *ms = CC(c).last_ms();
  });
}

int mrt_codec_read(mrt_codec* c, int which, void* dst, size_t bytes) {
  return guarded([&] {
    if (!dst) throw mrt::Error(MRT_ERR_INVALID, "null argument");
    auto [src, n] = CC(c).buffer(which);
    if (bytes != n) throw mrt::Error(MRT_ERR_INVALID, "codec_read: size mismatch (" + std::to_string(n) + " bytes)");
    MRT_HIP_CHECK(hipMemcpyAsync(dst, src, n, hipMemcpyDefault, CC(c).stream));
    MRT_HIP_CHECK(hipStreamSynchronize(CC(c).stream));
  });
}

void mrt_coca_config_default(mrt_coca_config* cfg) {
  if (!cfg) return;
  const mrt::CocaConfig k;
  cfg->d_model = k.d_model;
  cfg->num_heads = k.num_heads;
  cfg->d_head = k.d_head;
  cfg->d_ff = k.d_ff;
  cfg->num_layers = k.num_layers;
  cfg->pooler_d_head = k.pooler_d_head;
  cfg->vocab_size = k.vocab_size;
  cfg->max_text_len = k.max_text_len;
  cfg->rvq_depth = k.rvq_depth;
  cfg->codebook_size = k.codebook;
}

int mrt_coca_create(const char* encoder_path, const char* codebooks_path, const mrt_coca_config* cfg, int device,
                    mrt_coca** out) {
  return guarded([&] {
    if (!encoder_path || !codebooks_path || !cfg || !out) throw mrt::Error(MRT_ERR_INVALID, "null argument");
    *out = nullptr;
    const mrt::CocaConfig k = to_coca_config(cfg);
    mrt::SafetensorsFile enc(encoder_path), cbs(codebooks_path);
    auto h = std::make_unique<mrt_coca>();
    h->coca = std::make_unique<mrt::Coca>(enc, cbs, k, device);
    *out = h.release();
  });
}

int mrt_coca_create_from_tensors(int n, const char* const* names, const float* const* data,
                                 const int64_t* const* shapes, const int32_t* ndims, const mrt_coca_config* cfg,
                                 int device, mrt_coca** out) {
  return guarded([&] {
    if (!names || !data || !shapes || !ndims || !cfg || !out || n < 0)
      throw mrt::Error(MRT_ERR_INVALID, "null argument");
    *out = nullptr;
    const mrt::CocaConfig k = to_coca_config(cfg);
    mrt::TensorList src;
    for (int i = 0; i < n; ++i) {
      if (!names[i] || !data[i] || ndims[i] < 0) throw mrt::Error(MRT_ERR_INVALID, "bad tensor entry");
      src.add(names[i], data[i], std::vector<int64_t>(shapes[i], shapes[i] + ndims[i]));
    }
    auto h = std::make_unique<mrt_coca>();
    h->coca = std::make_unique<mrt::Coca>(src, src, k, device);
    *out = h.release();
  });
}

void mrt_coca_destroy(mrt_coca* h) { delete h; }

int mrt_coca_embed_text(mrt_coca* h, const int32_t* ids, const float* padding, float* embedding) {
  return guarded([&] {
    if (!ids || !padding || !embedding) throw mrt::Error(MRT_ERR_INVALID, "null argument");
    CO(h).embed_text(ids, padding, embedding);
  });
}

int mrt_coca_tokenize(mrt_coca* h, const float* embedding, int32_t* tokens) {
  return guarded([&] {
    if (!tokens) throw mrt::Error(MRT_ERR_INVALID, "null argument");
    CO(h).tokenize(embedding, tokens);
  });
}

int mrt_coca_style_tokens_lm(mrt_coca* h, const int32_t* ids, const float* padding, int style_depth,
                             int style_codebook_size, int vocab_style_offset, int32_t* out) {
  return guarded([&] {
    if (!ids || !padding || !out) throw mrt::Error(MRT_ERR_INVALID, "null argument");
    mrt::Coca& c = CO(h);
    if (style_depth < 0 || style_depth > c.cfg.rvq_depth)
      throw mrt::Error(MRT_ERR_INVALID, "style_tokens_lm: style_depth must be in [0, rvq_depth]");
    c.embed_text(ids, padding, nullptr);
    std::vector<int32_t> tok(c.cfg.rvq_depth);
    c.tokenize(nullptr, tok.data());
    for (int l = 0; l < style_depth; ++l) out[l] = vocab_style_offset + l * style_codebook_size + tok[l];
  });
}

int mrt_coca_embed_time(mrt_coca* h, float* ms) {
  return guarded([&] {
    if (!ms) throw mrt::Error(MRT_ERR_INVALID, "null argument");
    *ms = CO(h).last_ms();
  });
}

int mrt_coca_read(mrt_coca* h, int which, void* dst, size_t bytes) {
  return guarded([&] {
    if (!dst) throw mrt::Error(MRT_ERR_INVALID, "null argument");
    auto [src, n] = CO(h).buffer(which);
    if (bytes != n) throw mrt::Error(MRT_ERR_INVALID, "coca_read: size mismatch (" + std::to_string(n) + " bytes)");
    MRT_HIP_CHECK(hipMemcpyAsync(dst, src, n, hipMemcpyDefault, CO(h).stream));
    MRT_HIP_CHECK(hipStreamSynchronize(CO(h).stream));
  });
}

}  // extern "C"
