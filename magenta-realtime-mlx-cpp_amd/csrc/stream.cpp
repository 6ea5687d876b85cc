// Stream: the token half of System::generate_chunk (system.cpp:177-370) with
// the context resident on the device.  Between two chunks nothing crosses
// PCIe except the chunk's ids going out (and a style that changed coming in).
#include "stream.hpp"

#include <algorithm>
#include <random>

namespace mrt {

namespace {

const StreamConfig& checked(const Model& m, const StreamConfig& c) {
  const Config& mc = m.cfg;
  MRT_REQUIRE(c.chunk_frames >= 1 && c.chunk_frames <= c.context_frames,
              "stream: chunk_frames must be in [1, context_frames]");
  MRT_REQUIRE(c.levels == mc.rvq_depth, "stream: decoder_codec_rvq_depth must equal the model's rvq_depth");
  MRT_REQUIRE(c.enc_depth >= 0 && c.enc_depth <= c.levels, "stream: encoder_codec_rvq_depth must be in [0, levels]");
  MRT_REQUIRE(c.style_depth >= 0, "stream: encoder_style_rvq_depth must be >= 0");
  MRT_REQUIRE(c.enc_len() >= 1 && c.enc_len() <= mc.max_encoder_length,
              "stream: encoder length must be in [1, max_encoder_length]");
  MRT_REQUIRE(c.codebook >= 1 && c.codebook <= 1024, "stream: codebook_size must be in [1, 1024]");
  MRT_REQUIRE(c.codec_offset >= 0 && c.codec_offset + static_cast<int64_t>(c.codebook) * c.levels <= mc.vocab_size,
              "stream: codec levels exceed the vocabulary");
  MRT_REQUIRE(c.mask >= 0 && c.mask < mc.vocab_size, "stream: mask token out of range");
  MRT_REQUIRE(llm_to_rvq_roll_fits(c.context_frames, c.levels), "stream: context too large for the roll kernel");
  return c;
}

}  // namespace

Stream::Stream(Model& m, const StreamConfig& c) : cfg(checked(m, c)), st(m, 2, c.chunk_frames, c.enc_len()) {
  MRT_HIP_CHECK(hipSetDevice(m.device));
  const size_t nctx = static_cast<size_t>(c.context_frames) * c.levels;
  MRT_HIP_CHECK(hipMalloc(&d_ctx_, nctx * 4));
  MRT_HIP_CHECK(hipMalloc(&d_style_, std::max(c.style_depth, 1) * 4));
  MRT_HIP_CHECK(hipMalloc(&d_err_, 4));
  h_stage_n_ = std::max<size_t>(nctx, c.style_depth) + 1;
  MRT_HIP_CHECK(hipHostMalloc(&h_stage_, h_stage_n_ * 4, hipHostMallocDefault));
  // System::empty_state (system.cpp:165-176): every slot empty.
  std::fill(h_stage_, h_stage_ + nctx, -1);
  h_stage_[nctx] = 0;
  MRT_HIP_CHECK(hipMemcpyAsync(d_ctx_, h_stage_, nctx * 4, hipMemcpyHostToDevice, st.stream));
  MRT_HIP_CHECK(hipMemcpyAsync(d_err_, h_stage_ + nctx, 4, hipMemcpyHostToDevice, st.stream));
  MRT_HIP_CHECK(hipStreamSynchronize(st.stream));
  seed_base_ = (static_cast<uint64_t>(std::random_device{}()) << 32) ^ std::random_device{}();
}

Stream::~Stream() {
  (void)hipSetDevice(st.m.device);
  if (st.stream) (void)hipStreamSynchronize(st.stream);
  if (d_ctx_) (void)hipFree(d_ctx_);
  if (d_style_) (void)hipFree(d_style_);
  if (d_err_) (void)hipFree(d_err_);
  if (h_stage_) (void)hipHostFree(h_stage_);
  if (codec_ && codec_->stream) (void)hipStreamSynchronize(codec_->stream);
  for (void* q : {static_cast<void*>(d_codec_tok_), static_cast<void*>(d_audio_), static_cast<void*>(d_audio_out_),
                  static_cast<void*>(d_tail_)})
    if (q) (void)hipFree(q);
  if (h_audio_) (void)hipHostFree(h_audio_);
  if (ev_ctx_) (void)hipEventDestroy(ev_ctx_);
}

void Stream::attach_codec(Codec* c) {
  MRT_HIP_CHECK(hipSetDevice(st.m.device));
  if (codec_ && codec_->stream) MRT_HIP_CHECK(hipStreamSynchronize(codec_->stream));
  codec_ = nullptr;
  tail_valid_ = false;
  if (!c) return;
  const StreamConfig& k = cfg;
  MRT_REQUIRE(c->device == st.m.device, "attach_codec: the codec is on another device");
  MRT_REQUIRE(c->cfg.levels == k.levels && c->cfg.codebook == k.codebook,
              "attach_codec: the codec's rvq_levels / codebook_size differ from the stream's");
  MRT_REQUIRE(c->max_frames >= k.chunk_frames + k.crossfade_frames,
              "attach_codec: the codec's max_frames is below chunk_frames + crossfade_frames");
  MRT_REQUIRE(k.crossfade_frames >= 0 && k.crossfade_frames <= k.context_frames - k.chunk_frames,
              "attach_codec: crossfade_frames must fit in the context before the chunk");
  MRT_REQUIRE(k.samples_per_frame == c->cfg.samples_per_frame, "attach_codec: samples per frame differ");
  c->prepare(k.chunk_frames + k.crossfade_frames);  // geometry errors surface here, not mid-chunk
  const size_t nf = static_cast<size_t>(k.chunk_frames + k.crossfade_frames);
  const size_t T = nf * k.samples_per_frame;
  const size_t xf = static_cast<size_t>(k.crossfade_frames) * k.samples_per_frame;
  if (!d_codec_tok_) {
    MRT_HIP_CHECK(hipMalloc(&d_codec_tok_, nf * k.levels * 4));
    MRT_HIP_CHECK(hipMalloc(&d_audio_, T * 2 * 4));
    MRT_HIP_CHECK(hipMalloc(&d_audio_out_, std::max<size_t>(T - xf, 1) * 2 * 4));
    MRT_HIP_CHECK(hipMalloc(&d_tail_, std::max<size_t>(xf, 1) * 2 * 4));
    MRT_HIP_CHECK(hipHostMalloc(reinterpret_cast<void**>(&h_audio_), std::max<size_t>(T - xf, 1) * 2 * 4,
                                hipHostMallocDefault));
    MRT_HIP_CHECK(hipEventCreateWithFlags(&ev_ctx_, hipEventDisableTiming));
  }
  codec_ = c;
}

// d_style_ <- style (only when it differs from what the device holds).
void Stream::upload_style(const int32_t* style) {
  const int s = cfg.style_depth;
  if (style_set_ && std::equal(style, style + s, dev_style_.begin())) return;
  MRT_HIP_CHECK(hipStreamSynchronize(st.stream));  // staging reuse
  std::copy(style, style + s, h_stage_);
  MRT_HIP_CHECK(hipMemcpyAsync(d_style_, h_stage_, static_cast<size_t>(s) * 4, hipMemcpyHostToDevice, st.stream));
  MRT_HIP_CHECK(hipStreamSynchronize(st.stream));
  dev_style_.assign(style, style + s);
  style_set_ = true;
}

// Encoder inputs from the device context and the style (null: masked), then
// the encoder and cross K/V, all enqueued on the state's stream.
void Stream::build_and_encode(const int32_t* style) {
  const StreamConfig& c = cfg;
  if (style) upload_style(style);
  encoder_inputs(d_ctx_, c.context_frames, c.levels, c.enc_depth, style ? d_style_ : nullptr, c.style_depth,
                 c.codebook, c.codec_offset, c.mask, st.enc_tokens_dev(), st.stream);
  st.encode_device();
}

// The decode options of a chunk (GenerateChunkOptions -> GenerateOptions,
// system.cpp:236-260).
GenOpts Stream::gen_opts(const ChunkOpts& o) const {
  const StreamConfig& c = cfg;
  MRT_REQUIRE(o.speculative >= 0 && o.speculative <= 2, "generate_chunk: speculative must be 0, 1 or 2");
  GenOpts g;
  g.num_frames = c.chunk_frames;
  g.rvq_depth = c.levels;
  g.temperature = o.temperature;
  g.top_k = o.top_k;
  g.guidance_weight = o.guidance_weight;
  g.seed = o.has_seed ? o.seed : seed_base_ + static_cast<uint64_t>(chunk_index);
  g.codebook = c.codebook;
  g.codec_offset = c.codec_offset;
  g.teacher = o.teacher;
  g.use_graph = o.use_graph;
  g.speculative = o.speculative != 0;
  return g;
}

void Stream::compile(const ChunkOpts& o) {
  MRT_HIP_CHECK(hipSetDevice(st.m.device));
  // the encoder inputs of the current context (masked style) and the encoder
  // itself run once too, unless a pipelined encoder output must be kept
  if (!pre_valid_) build_and_encode(nullptr);
  st.compile(gen_opts(o));
}

// Encoder (or the pipelined one), decode, llm_to_rvq and the roll; returns
// with the state's stream idle.
void Stream::token_half(const int32_t* style, const ChunkOpts& o, int32_t* llm_out, int32_t* rvq_out) {
  const StreamConfig& c = cfg;
  const int vocab = st.m.cfg.vocab_size;
  MRT_HIP_CHECK(hipSetDevice(st.m.device));
  if (style)
    for (int i = 0; i < c.style_depth; ++i)
      MRT_REQUIRE(style[i] >= 0 && style[i] < vocab, "generate_chunk: style token out of range");

  // Pipelined encoder output of the previous call, valid when the style
  // matches (the context can only have changed through set_context, which
  // drops it) -- the fingerprint check of system.cpp:218-232.
  const bool reuse = pre_valid_ && (style ? (!pre_masked_ && std::equal(style, style + c.style_depth, pre_style_.begin()))
                                          : pre_masked_);
  pre_valid_ = false;
  if (!reuse) build_and_encode(style);

  GenOpts g = gen_opts(o);
  g.speculative = o.speculative == 1 || (o.speculative == 2 && spec_pause_ == 0);
  if (o.speculative == 2 && !spec_full_) g.spec_frames = kSpecProbeFrames;  // a probe
  const size_t n = static_cast<size_t>(c.chunk_frames) * c.levels;
  llm_tmp_.resize(n);
  st.generate(nullptr, g, llm_tmp_.data());  // waits for the chunk's ids
  if (o.speculative == 2) {
    if (spec_pause_ > 0) {
      --spec_pause_;
    } else {
      const float acc = st.spec_acceptance();  // -1: no drafts yet (first chunk)
      if (acc >= kSpecMinAcceptance) {
        spec_full_ = true;
        spec_backoff_ = kSpecPause;
      } else if (acc >= 0.f) {
        spec_full_ = false;
        spec_pause_ = spec_backoff_;
        spec_backoff_ = std::min(2 * spec_backoff_, kSpecMaxPause);
      }
    }
  }
  if (llm_out) std::copy(llm_tmp_.begin(), llm_tmp_.end(), llm_out);

  // llm_to_rvq (system.cpp:289-292) and the context roll (system.cpp:315-333).
  llm_to_rvq_roll(st.tokens_dev(), c.chunk_frames, c.levels, c.codebook, c.codec_offset, d_ctx_, c.context_frames,
                  d_err_, st.stream);
  const size_t tail = static_cast<size_t>(c.context_frames - c.chunk_frames) * c.levels;
  MRT_HIP_CHECK(hipMemcpyAsync(h_stage_, d_ctx_ + tail, n * 4, hipMemcpyDeviceToHost, st.stream));
  MRT_HIP_CHECK(hipMemcpyAsync(h_stage_ + n, d_err_, 4, hipMemcpyDeviceToHost, st.stream));
  MRT_HIP_CHECK(hipStreamSynchronize(st.stream));
  if (h_stage_[n] != 0) {
    h_stage_[n] = 0;
    MRT_HIP_CHECK(hipMemcpyAsync(d_err_, h_stage_ + n, 4, hipMemcpyHostToDevice, st.stream));
    MRT_HIP_CHECK(hipStreamSynchronize(st.stream));
    throw Error(1, "llm_to_rvq: token levels do not match expected RVQ structure");
  }
  if (rvq_out) std::copy(h_stage_, h_stage_ + n, rvq_out);
}

// Next chunk's encoder kicked off before returning (system.cpp:334-370).
void Stream::kick_pipeline(const int32_t* style) {
  build_and_encode(style);
  pre_valid_ = true;
  pre_masked_ = style == nullptr;
  if (style) pre_style_.assign(style, style + cfg.style_depth);
}

void Stream::generate_chunk(const int32_t* style, const ChunkOpts& o, int32_t* llm_out, int32_t* rvq_out) {
  token_half(style, o, llm_out, rvq_out);
  if (o.pipeline_encoder) kick_pipeline(style);
  tail_valid_ = false;  // this chunk's audio was not made: no tail for the next crossfade
  ++chunk_index;
}

void Stream::generate_chunk_audio(const int32_t* style, const ChunkOpts& o, int32_t* llm_out, int32_t* rvq_out,
                                  float* audio_out) {
  MRT_REQUIRE(codec_ != nullptr, "generate_chunk_audio: no codec attached");
  MRT_REQUIRE(audio_out != nullptr, "generate_chunk_audio: null audio buffer");
  const StreamConfig& c = cfg;
  const bool first = chunk_index == 0;
  token_half(style, o, llm_out, rvq_out);
  // decoder input from the rolled context, then the codec on its own stream
  const int nf = c.chunk_frames + c.crossfade_frames;
  codec_frames(d_ctx_, c.context_frames, c.levels, c.chunk_frames, c.crossfade_frames, first, d_codec_tok_,
               st.stream);
  MRT_HIP_CHECK(hipEventRecord(ev_ctx_, st.stream));
  MRT_HIP_CHECK(hipStreamWaitEvent(codec_->stream, ev_ctx_, 0));
  codec_->decode_device(d_codec_tok_, nf, d_audio_);
  const int T = nf * c.samples_per_frame, xf = c.crossfade_frames * c.samples_per_frame;
  // system.cpp:423-425: the ramp needs a previous tail of the same length
  crossfade(d_audio_, T, xf, !first && tail_valid_ && xf > 0 && T - xf >= xf, d_tail_, d_audio_out_, codec_->stream);
  const size_t na = static_cast<size_t>(T - xf) * 2;
  MRT_HIP_CHECK(hipMemcpyAsync(h_audio_, d_audio_out_, na * 4, hipMemcpyDeviceToHost, codec_->stream));
  // the next chunk's encoder runs on the state's stream while the codec runs
  if (o.pipeline_encoder) kick_pipeline(style);
  MRT_HIP_CHECK(hipStreamSynchronize(codec_->stream));
  std::copy(h_audio_, h_audio_ + na, audio_out);
  tail_valid_ = xf > 0;
  ++chunk_index;
}


void Stream::set_context(const int32_t* ctx_host, int64_t index) {
  const StreamConfig& c = cfg;
  const size_t nctx = static_cast<size_t>(c.context_frames) * c.levels;
  for (size_t i = 0; i < nctx; ++i)
    MRT_REQUIRE(ctx_host[i] >= -1 && ctx_host[i] < c.codebook, "set_context: code out of range [-1, codebook)");
  MRT_REQUIRE(index >= 0, "set_context: chunk index must be >= 0");
  MRT_HIP_CHECK(hipSetDevice(st.m.device));
  MRT_HIP_CHECK(hipStreamSynchronize(st.stream));
  std::copy(ctx_host, ctx_host + nctx, h_stage_);
  MRT_HIP_CHECK(hipMemcpyAsync(d_ctx_, h_stage_, nctx * 4, hipMemcpyHostToDevice, st.stream));
  MRT_HIP_CHECK(hipStreamSynchronize(st.stream));
  chunk_index = index;
  pre_valid_ = false;
  tail_valid_ = false;
}

void Stream::get_context(int32_t* ctx_host, int64_t* index) {
  const size_t nctx = static_cast<size_t>(cfg.context_frames) * cfg.levels;
  MRT_HIP_CHECK(hipSetDevice(st.m.device));
  if (ctx_host) {
    MRT_HIP_CHECK(hipStreamSynchronize(st.stream));
    MRT_HIP_CHECK(hipMemcpyAsync(h_stage_, d_ctx_, nctx * 4, hipMemcpyDeviceToHost, st.stream));
    MRT_HIP_CHECK(hipStreamSynchronize(st.stream));
    std::copy(h_stage_, h_stage_ + nctx, ctx_host);
  }
  if (index) *index = chunk_index;
}

}  // namespace mrt
