// A stream's token context on the device: System::generate_chunk's LLM half
// (system.cpp:177-333) without host round trips between chunks.
#pragma once

#include <cstdint>
#include <vector>

#include "codec.hpp"
#include "common.hpp"
#include "model.hpp"

namespace mrt {

// Encoder inputs (2, frames * e + s) int32 from the context (frames, levels)
// (system.cpp:62-95); style may be null (every style slot MASK).
void encoder_inputs(const int* ctx, int frames, int levels, int e, const int* style, int s, int C, int offset,
                    int mask, int* out, hipStream_t st);

// LLM ids (n, levels) -> RVQ codes (rvq.cpp:112-132, safe: *err = 1 on a
// level mismatch, context untouched), rolled into the context
// (frames, levels) in place (system.cpp:320-333).
bool llm_to_rvq_roll_fits(int frames, int levels);
void llm_to_rvq_roll(const int* llm, int n, int levels, int C, int offset, int* ctx, int frames, int* err,
                     hipStream_t st);

// The codec input (n + xf, levels) of a chunk from the rolled context
// (system.cpp:294-313); first: the crossfade rows are zeros.
void codec_frames(const int* ctx, int frames, int levels, int n, int xf, bool first, int* out, hipStream_t st);
// Crossfade (system.cpp:410-437) of audio (T, 2) against tail (xf, 2) into
// out (T - xf, 2); tail <- audio's last xf samples.
void crossfade(const float* audio, int T, int xf, bool fade, float* tail, float* out, hipStream_t st);

// The SystemConfig fields the token half reads (system.h:44-83).
struct StreamConfig {
  int chunk_frames = 50;       // chunk_length_frames
  int context_frames = 250;    // context_length_frames
  int codebook = 1024;         // codec_rvq_codebook_size
  int enc_depth = 4;           // encoder_codec_rvq_depth
  int style_depth = 6;         // encoder_style_rvq_depth
  int levels = 16;             // decoder_codec_rvq_depth
  int mask = 1;                // vocab_mask_token
  int codec_offset = 2;        // vocab_codec_offset
  int crossfade_frames = 1;    // crossfade_length_frames (0.04 s at 25 Hz)
  int samples_per_frame = 1920;  // codec_sample_rate / codec_frame_rate
  int enc_len() const { return context_frames * enc_depth + style_depth; }
};

// GenerateChunkOptions (system.h:86-121).
struct ChunkOpts {
  float temperature = 1.1f;
  int top_k = 40;
  float guidance_weight = 5.0f;
  bool has_seed = false;
  uint64_t seed = 0;
  bool pipeline_encoder = false;
  bool use_graph = true;
  const int32_t* teacher = nullptr;  // host (chunk_frames, levels) ids fed in place of the draws
  // Speculative depth decoding, drafts = the previous chunk's tokens of the
  // same frame: 0 off, 1 on, 2 adaptive: a chunk speculates only its first
  // kSpecProbeFrames frames (the rest decodes plainly); when at least
  // kSpecMinAcceptance of the probed levels came from the verification pass,
  // whole chunks speculate while their acceptance stays at or above it.  After
  // a probe or chunk below it, kSpecPause chunks decode plainly before the
  // next probe, doubling after each further miss up to kSpecMaxPause.
  int speculative = 0;
};

// SystemState's token context (system.h:124-160) resident in device memory,
// with the decode state it feeds.  Each chunk: encoder inputs built on the
// device from the context and style, encoder, decode, LLM ids -> RVQ codes
// rolled into the context; with pipeline_encoder the next chunk's encoder is
// enqueued before returning (system.cpp:334-370) and reused when the next
// call's style matches.
constexpr float kSpecMinAcceptance = 0.25f;
constexpr int kSpecPause = 4;
constexpr int kSpecMaxPause = 64;
constexpr int kSpecProbeFrames = 2;

class Stream {
 public:
  Stream(Model& m, const StreamConfig& cfg);
  ~Stream();
  Stream(const Stream&) = delete;
  Stream& operator=(const Stream&) = delete;

  StreamConfig cfg;
  State st;
  int64_t chunk_index = 0;

  // style: host (style_depth) ids or null (masked).  llm_out / rvq_out: host
  // (chunk_frames, levels) or null.
  void generate_chunk(const int32_t* style, const ChunkOpts& o, int32_t* llm_out, int32_t* rvq_out);
  // compile_for_inference for this stream's chunks (State::compile with the
  // chunk's decode options); the context and chunk index are not touched.
  void compile(const ChunkOpts& o);
  // The whole System::generate_chunk (system.cpp:177-440): the token half,
  // then the codec decode of [the crossfade frame, the chunk] on the attached
  // codec's stream (overlapping the pipelined encoder of the next chunk) and
  // the crossfade.  audio_out: host (chunk_frames * samples_per_frame, 2).
  void generate_chunk_audio(const int32_t* style, const ChunkOpts& o, int32_t* llm_out, int32_t* rvq_out,
                            float* audio_out);
  // Not owned; null detaches.  Its levels / codebook must be the stream's and
  // its max_frames >= chunk_frames + crossfade_frames.
  void attach_codec(Codec* c);
  void set_context(const int32_t* ctx_host, int64_t index);  // (context_frames, levels), -1 = empty
  void get_context(int32_t* ctx_host, int64_t* index);
  bool pre_encoded() const { return pre_valid_; }

 private:
  void upload_style(const int32_t* style);
  void build_and_encode(const int32_t* style);
  void token_half(const int32_t* style, const ChunkOpts& o, int32_t* llm_out, int32_t* rvq_out);
  GenOpts gen_opts(const ChunkOpts& o) const;
  void kick_pipeline(const int32_t* style);
  Codec* codec_ = nullptr;
  int* d_codec_tok_ = nullptr;
  float *d_audio_ = nullptr, *d_audio_out_ = nullptr, *d_tail_ = nullptr, *h_audio_ = nullptr;
  bool tail_valid_ = false;  // d_tail_ holds the previous chunk's tail (crossfade applies)
  hipEvent_t ev_ctx_ = nullptr;
  int* d_ctx_ = nullptr;
  int* d_style_ = nullptr;
  int* d_err_ = nullptr;
  int32_t* h_stage_ = nullptr;  // pinned: style in, codes and flag out
  size_t h_stage_n_ = 0;
  bool style_set_ = false;            // d_style_ holds dev_style_
  std::vector<int32_t> dev_style_;
  bool pre_valid_ = false;            // st holds the encoder output of the context + pre_style_
  bool pre_masked_ = true;
  std::vector<int32_t> pre_style_;
  std::vector<int32_t> llm_tmp_;
  uint64_t seed_base_ = 0;
  int spec_pause_ = 0;          // adaptive speculation: chunks left to decode plainly
  int spec_backoff_ = kSpecPause;  // the pause after the next miss
  bool spec_full_ = false;     // the last speculation met kSpecMinAcceptance: whole chunks
};

}  // namespace mrt
