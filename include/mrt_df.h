/*
 * mrt_df.h -- C ABI of the MI355X (gfx950) Depthformer streaming-decode backend.
 *
 * Drop-in for the Depthformer hot path of magenta-realtime-mlx-cpp: the
 * `Depthformer::{encode, temporal_step, depth_step}` methods, the `.mlxfn`
 * imported-function ABI they dispatch to, and the `generate_tokens` 50x16
 * block-autoregressive loop.  Citations are to files of that project.
 *
 * Conventions
 *   - Every function returns MRT_OK (0) or an error code; the message of the
 *     last error on the calling thread is `mrt_last_error()`.  No C++
 *     exception crosses this boundary (the reference throws
 *     std::runtime_error / std::out_of_range at the same places).
 *   - Activation tensors passed to step functions are DEVICE pointers in the
 *     model dtype (fp32 or bf16 raw bits) on the handle's device; logits are
 *     fp32 device buffers.  Token arrays are HOST int32.
 *   - A model handle owns the weights; a state handle owns one decode stream's
 *     encoder output, cross-attention K/V, ring KV caches, scratch and HIP
 *     stream.  Calls on one state are not thread-safe; distinct states may be
 *     driven from distinct threads.  Their persistent kernels (one workgroup
 *     per CU) never run side by side: each decode or step launch of a state
 *     waits on the device for the previous one of any state on that device
 *     (and so do the hand-off probes below).  This ordering holds among the
 *     calls of one process: persistent work of two processes sharing a GPU
 *     is not ordered by this library.
 */
#ifndef MRT_DF_H_
#define MRT_DF_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MRT_OK 0
#define MRT_ERR_INVALID 1     /* bad argument / shape / cache length   */
#define MRT_ERR_STATE 2       /* call order violated (e.g. no encoder)  */
#define MRT_ERR_HIP 3         /* HIP runtime failure                    */
#define MRT_ERR_MISSING_KEY 4 /* weight bundle lacks a tensor           */
#define MRT_ERR_FORMAT 5      /* malformed bundle                       */
#define MRT_ERR_INTERNAL 6

/* Model storage dtypes: the reference's fp32 | bf16 | fp16 (dtype.cpp:35-49). */
#define MRT_DTYPE_F32 0
#define MRT_DTYPE_BF16 1
#define MRT_DTYPE_F16 2

/* DepthformerConfig (src/magenta_realtime_mlx/depthformer/model.h:47-68). */
typedef struct mrt_df_config {
  int32_t vocab_size;
  int32_t d_model;
  int32_t d_kv;
  int32_t d_ff;
  int32_t num_heads;
  int32_t num_encoder_layers;
  int32_t num_temporal_layers;
  int32_t num_depth_layers;
  int32_t max_encoder_length;
  int32_t rvq_depth;
  int32_t temporal_num_buckets;
  int32_t temporal_max_distance;
  int32_t depth_num_buckets;
  int32_t depth_max_distance;
} mrt_df_config;

/* GenerateOptions (depthformer/decode.h:48-57) plus the vocabulary layout
 * of SystemConfig (system.h:44-83) that build_vocab_masks encodes
 * (system.cpp:135-157). */
typedef struct mrt_gen_opts {
  int32_t num_frames;      /* 50 */
  int32_t rvq_depth;       /* 16 */
  float temperature;       /* 1.1; 0 -> argmax */
  int32_t top_k;           /* 40; <= 0 -> no top-k */
  float guidance_weight;   /* 5.0 streaming, 4.0 GenerateOptions default */
  uint64_t seed;           /* per-chunk seed (base seed + chunk index) */
  int32_t codebook_size;   /* 1024 */
  int32_t codec_offset;    /* 2 */
  const int32_t* teacher;  /* optional host (num_frames, rvq_depth) ids fed back instead of draws */
  int32_t use_graph;       /* replay the decode loop from a captured hipGraph */
  /* Optional DEVICE buffers filled during the loop (parity / inspection): */
  float* record_slices;    /* (F, L, rows, codebook) level-slice logits (fp32) */
  void* record_temporal;   /* (F, rows, d_model) temporal_step outputs (model dtype) */
  int32_t* record_drawn;   /* (F, L) the model's own draws (device) */
  void* record_frame_mean; /* (F, rows, d_model) mean of each frame's 16 level embeddings */
  /* GenerateOptions speculative path (decode.cpp:150-237, 380-446): frame f's
   * levels are drafted with the previous call's tokens of frame f, verified in
   * one causal pass over the frame's 16 positions, accepted up to the first
   * disagreement (whose draw is the token), the rest decoded as usual.  The
   * tokens are those of the same draws from the same logits.  bf16 models on
   * the persistent path; ignored (plain decode) on a state's
   * first call, when num_frames differs from the previous call's, with a
   * teacher, or with record_drawn / record_frame_mean.  Any nonzero value
   * turns it on (the adaptive mode 2 is a policy of the stream entry points). */
  int32_t speculative;
} mrt_gen_opts;

typedef struct mrt_df mrt_df;
typedef struct mrt_df_state mrt_df_state;

/* Thread-local message of the last failing call ("" when none). */
const char* mrt_last_error(void);

/* DepthformerConfig::base() / ::large() (depthformer/model.cpp:34-48). */
void mrt_df_config_base(mrt_df_config* cfg);
void mrt_df_config_large(mrt_df_config* cfg);

/* Depthformer::Depthformer(bundle, config, dtype) (model.cpp:173-213) with
 * WeightBundle loading (weights.cpp:118-133): reads the fp32 .safetensors
 * bundle (key layout model.cpp:177-198, modules.cpp:342-381), casts to
 * `dtype`, repacks and uploads to `device`. */
int mrt_df_create(const char* bundle_path, const mrt_df_config* cfg, int dtype, int device,
                  mrt_df** out);
/* Same, from caller-owned fp32 host arrays named with the bundle keys. */
int mrt_df_create_from_tensors(int n, const char* const* names, const float* const* data,
                               const int64_t* const* shapes, const int32_t* ndims,
                               const mrt_df_config* cfg, int dtype, int device, mrt_df** out);
void mrt_df_destroy(mrt_df* h);
int mrt_df_get_config(const mrt_df* h, mrt_df_config* cfg, int* dtype);

/* Per-stream state: rows = 2 (CFG pair) per stream; KV rings sized for
 * `max_frames` temporal steps and cfg.rvq_depth depth steps; encoder
 * length `enc_len` (<= max_encoder_length).  Replaces the caller-owned
 * std::vector<LayerCache> of empty_{temporal,depth}_cache (model.cpp:280-300). */
int mrt_df_state_create(mrt_df* h, int rows, int max_frames, int enc_len, mrt_df_state** out);
void mrt_df_state_destroy(mrt_df_state* st);
/* The state's hipStream_t (all work of the state is ordered on it). */
int mrt_df_state_stream(mrt_df_state* st, void** hip_stream);
int mrt_df_sync(mrt_df_state* st);

/* Depthformer::encode (model.cpp:226-241): tokens (rows, enc_len) host int32
 * -> encoder output, then the cross-attention K/V of every temporal layer
 * (DecoderLayer::precompute_cross_kv, modules.cpp:448-455), kept in the state. */
int mrt_df_encode(mrt_df_state* st, const int32_t* tokens);

/* Depthformer::temporal_step (model.cpp:322-514): frame_emb (rows, d_model)
 * device, model dtype -> out (rows, d_model) (no final norm).  If
 * `enc_out` is non-null and frame_idx == 0, the cross K/V are projected from
 * it first (the eager frame-0 path, modules.cpp:397-404); otherwise those of
 * the last mrt_df_encode are used.  The temporal cache must hold exactly
 * frame_idx entries (it is reset by frame_idx == 0). */
int mrt_df_temporal_step(mrt_df_state* st, const void* frame_emb, const void* enc_out,
                         int frame_idx, void* out);

/* Depthformer::depth_step (model.cpp:516-659): tok_emb (rows, d_model) device
 * -> logits.  level < 0: full vocabulary (rows, vocab_size) fp32 (the
 * reference's return value); level >= 0: only lm_head rows
 * [codec_offset + codebook*level, +codebook) as (rows, codebook) fp32 --
 * exact under the level's vocabulary mask (system.cpp:135-157).  The depth
 * cache must hold exactly depth_idx entries (reset by depth_idx == 0). */
int mrt_df_depth_step(mrt_df_state* st, const void* tok_emb, int depth_idx, int level,
                      int codebook_size, int codec_offset, float* logits);

/* The two steps with the reference's optional `position_bias` argument
 * (temporal_step / depth_step, model.cpp:322-330, 516-525): position_bias is a
 * DEVICE (num_heads, idx + 1) model-dtype array -- the reference's
 * (1, H, 1, idx + 1) -- used instead of the rel-pos bias of the state's
 * tables; idx is frame_idx / depth_idx.  Otherwise as mrt_df_temporal_step /
 * mrt_df_depth_step. */
int mrt_df_temporal_step_with_bias(mrt_df_state* st, const void* frame_emb, const void* enc_out, int frame_idx,
                                   const void* position_bias, void* out);
int mrt_df_depth_step_with_bias(mrt_df_state* st, const void* tok_emb, int depth_idx, const void* position_bias,
                                int level, int codebook_size, int codec_offset, float* logits);

/* Depthformer::token_embedding() (depthformer/model.h:127) applied to ids,
 * as the decode loop embeds every fed token (decode.cpp:366-368, 476-477;
 * Embedding::operator(), modules.cpp:110-112): writes the n rows
 * emb[ids[i]] -- (n, d_model) model dtype -- to the DEVICE buffer `out`.
 * ids: host int32, each in [0, vocab_size) (else MRT_ERR_INVALID, nothing
 * written).  Enqueued on `hip_stream` (NULL = the null stream); waits for it. */
int mrt_df_embed_tokens(mrt_df* h, const int32_t* ids, int n, void* out, void* hip_stream);

/* Depthformer::position_embedding(seq_len) (model.cpp:215-224): the first
 * seq_len rows of the fp32 sinusoid table (model.cpp:54-80) as DEVICE fp32
 * (seq_len, d_model).  seq_len > max_encoder_length fails with
 * MRT_ERR_INVALID "seq_len exceeds max_encoder_length" (the reference's
 * std::out_of_range).  Synchronous. */
int mrt_df_position_embedding(mrt_df* h, int seq_len, float* out);

/* Depthformer::precompute_temporal_biases / precompute_depth_biases
 * (model.cpp:302-320): kind 0 = temporal, 1 = depth.  Writes the biases of
 * steps 0..n-1 back to back into `out` (DEVICE, model dtype,
 * num_heads * n * (n + 1) / 2 elements): step f's (num_heads, f + 1) block --
 * the reference's f-th (1, H, 1, f + 1) array -- starts at element
 * num_heads * f * (f + 1) / 2, so `out + that` is step f's position_bias.
 * Waits for the result. */
int mrt_df_precompute_biases(mrt_df* h, int kind, int n, void* out);

/* Empties the state's temporal (kind 0) or depth (kind 1) KV cache, as
 * replacing it with empty_temporal_cache() / empty_depth_cache() does in the
 * reference (model.cpp:275-300): the next step of that kind must be at index 0.
 * The cross-attention K/V of the last encode stay. */
int mrt_df_state_reset_cache(mrt_df_state* st, int kind);

/* generate_tokens (depthformer/decode.cpp:239-573), with the speculative
 * path of decode.cpp:380-446 when opts->speculative applies:
 * enc_tokens (rows, enc_len) host int32 (NULL: reuse the last encode) ->
 * out_tokens (num_frames, rvq_depth) host int32 LLM ids.  CFG, level mask,
 * temperature/top-k sampling, token feedback and the frame mean all run on
 * the device; the host syncs once at the end. */
int mrt_df_generate_tokens(mrt_df_state* st, const int32_t* enc_tokens, const mrt_gen_opts* opts,
                           int32_t* out_tokens);

/* One draw of the decode loop (decode.cpp:465-474): cfg_combine
 * (decode.cpp:71-85) of rows 0/1 of `slice` (device fp32, (2, codebook) --
 * one level's logits, i.e. apply_vocab_mask of decode.cpp:87-91 already
 * applied by slicing), then sample_with_temperature (decode.cpp:124-148):
 * argmax at temperature 0, else top_k_logits (ties at the threshold kept,
 * decode.cpp:104-122) and a categorical draw by Gumbel-max with Philox noise
 * keyed by (seed, frame, level, candidate).  Writes the LLM id
 * codec_offset + codebook*level + index to *token (host). */
int mrt_df_sample_level(mrt_df_state* st, const float* slice, const mrt_gen_opts* opts, int frame,
                        int level, int32_t* token);
/* No counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture, serving loops that forbid it).  The
 * draw of mrt_df_sample_level without a state: `slice_dev` is the same
 * (2, codebook) fp32 DEVICE array, the LLM id goes to token_dev[0] (DEVICE
 * int32), the work is enqueued on `hip_stream` (a hipStream_t of the model's
 * device; NULL = the null stream) and the call returns without waiting.  The
 * seed travels by value in the kernel arguments.  The fed-back embedding rows
 * the draw kernel also writes (discarded here) live in a fixed 32 KiB device
 * array of the library (one per device, held until the process ends), so
 * d_model * element size * 6 + 256 must be <= 32768 (fp32: d_model <= 1354;
 * bf16: the draw kernel's own limit, 2048), else MRT_ERR_INVALID.  Calls that
 * overlap on one device share that array, but each still writes the token of
 * its own slice, seed, frame and level.  Allocates nothing; shares the draw
 * kernel of mrt_df_sample_level, so tokens are identical. */
int mrt_df_sample_level_noalloc(mrt_df* h, const float* slice_dev, const mrt_gen_opts* opts, int frame, int level,
                                int32_t* token_dev, void* hip_stream);

/* Depthformer::depth_forward_full (depthformer/model.cpp:243-268, model.h:94):
 * the depth decoder as one pass over k_len positions (1..rvq_depth) of both
 * CFG rows, decoder_norm and lm_head.  token_embeddings: DEVICE (2, k_len,
 * d_model) model dtype.  position_bias: NULL for the rel-pos bias of the
 * k_len x k_len block at query offset 0 (the reference's default), or DEVICE
 * (num_heads, k_len, k_len) model dtype -- the reference's (1, H, k, k).
 * causal != 0 masks keys after the query (modules.cpp:197-209).  Writes
 * DEVICE fp32 (2, k_len, vocab_size) logits (each rounded to the model dtype,
 * as lm_head's output).  The state's caches are not touched; waits for the
 * result. */
int mrt_df_depth_forward_full(mrt_df_state* st, const void* token_embeddings, int k_len, const void* position_bias,
                              int causal, float* logits);

/* Instrumentation, no counterpart in the reference (its CLI times whole
 * chunks on the host, cli/main.cpp:459-505): GPU time in ms of the decode
 * section of the last mrt_df_generate_tokens call on this state -- the
 * Gumbel noise table and the decode launches after the encoder -- from HIP
 * events recorded on the state's stream.  *launches (may be NULL) receives
 * the number of persistent-kernel launches in it: num_frames with the frame
 * kernel, num_frames * (1 + rvq_depth) with one launch per step, 0 on the
 * per-layer path.  Waits for the section to finish. */
int mrt_df_state_decode_time(mrt_df_state* st, float* ms, int* launches);
/* Depthformer::compile_for_inference (model.cpp:697-...), per state: prepares
 * the decode for `opts` before the first real call, so that call pays no
 * one-time work.  Builds the layer-0 q/k/v table for the options' codebook and
 * codec offset, captures and instantiates the decode graph (opts->use_graph;
 * with opts->speculative the speculative graph as well) and launches every
 * kernel of the path once, through untimed decodes on the state's encoder
 * output (on an encoding of PAD ids when there is none, which is then
 * dropped: encode or pass enc_tokens before generating).  opts->teacher and
 * the record buffers are ignored.  The KV caches and the speculative draft
 * history are left as before the call; waits for the work. */
int mrt_df_state_compile(mrt_df_state* st, const mrt_gen_opts* opts);

/* The per-chunk split of the reference's MRT_PROFILE_DECODE breakdown
 * (decode.cpp:36-49, 529-565) for the last mrt_df_generate_tokens call on a
 * state, in GPU milliseconds.  total_ms is mrt_df_state_decode_time's figure;
 * encoder_ms the state's last encoder pass (-1 if none was timed); bias_ms 0
 * (the rel-pos biases are precomputed once per model); temporal_ms / depth_ms
 * / sample_ms sum over the frames the temporal step, the 16 depth steps with
 * their head logits, and the draws (CFG, top-k, sampling, embedding feedback),
 * from workgroup 0's device wall-clock stamps inside the frame kernel, taken
 * only while profiling is on (MRT_PROFILE_DECODE non-empty when the state is
 * created, or mrt_df_state_set_profile); -1 when the last call took none (the
 * per-step and speculative paths).  frames = the frames stamped. */
typedef struct mrt_decode_profile {
  float total_ms;
  float encoder_ms;
  float bias_ms;
  float temporal_ms;
  float depth_ms;
  float sample_ms;
  int32_t frames;
} mrt_decode_profile;
/* Turns the frame kernel's phase stamps on or off for later decodes. */
int mrt_df_state_set_profile(mrt_df_state* st, int on);
/* Waits for the last decode; fills *out.  MRT_ERR_INVALID before any decode. */
int mrt_df_state_decode_profile(mrt_df_state* st, mrt_decode_profile* out);

/* Instrumentation, no counterpart in the reference: with MRT_TRACE_PHASES set
 * when the state was created, the persistent kernels' workgroup 0 stamps the
 * device wall clock at every phase boundary of frame 1 of a decode (its
 * temporal step, then depth level 1).  Copies the 2 x 512 raw stamps of the
 * last decode into `out` (n >= 1024 words; zero = not reached) and the clock
 * rate in MHz into *clock_mhz.  MRT_ERR_INVALID when tracing is off. */
int mrt_df_state_phase_trace(mrt_df_state* st, uint64_t* out, int n, float* clock_mhz);
/* Share of the last mrt_df_generate_tokens call's RVQ levels whose token came
 * from the speculative verification pass (accepted drafts plus each frame's
 * first disagreement); -1 when that call did not speculate.  No counterpart
 * in the reference. */
int mrt_df_state_spec_acceptance(mrt_df_state* st, float* acceptance);

/* Measurement, no counterpart in the reference: the device's read bandwidth
 * in GB/s (1e9 B/s) for a `bytes` buffer (>= 1 MiB, multiple of 16) read
 * `passes` times (1..1000) after one warm pass, timed with HIP events.  A
 * buffer well below the 256 MB last-level cache of MI355X measures that cache
 * (the MALL); one of several GB measures HBM.  Allocates and frees the buffer;
 * for the benchmark's roofline peaks. */
int mrt_probe_read_bandwidth(int device, size_t bytes, int passes, float* gbps);

/* Measurement, no counterpart in the reference: the latency floor of one phase
 * hand-off of the persistent kernels.  mrt_probe_handoff: microseconds per
 * round of an all-gather of `words` (workgroups..1024, a multiple of
 * `workgroups`, at most 256 per workgroup) tagged 64-bit words among
 * `workgroups` (1..CU count) workgroups -- each stores its share with
 * agent-scope atomics, waits `delay` (0..256) rounds of s_sleep(1) (64 clocks
 * each), then polls all words -- over `rounds` (1..100000) rounds.  mrt_probe_pingpong: one-way microseconds of a word bounced
 * `rounds` times between workgroups 0 and `peer` (1..CU count - 1).  Both
 * allocate and free a 16 KiB buffer; every poll is bounded (a spin limit
 * returns MRT_ERR_HIP). */
int mrt_probe_handoff(int device, int workgroups, int words, int rounds, int delay, float* us_per_round);
int mrt_probe_pingpong(int device, int peer, int rounds, float* us_one_way);

/* State buffers exposed for parity checks (device-to-device copies). */
#define MRT_BUF_ENC_OUT 0     /* (rows, enc_len, d_model)                       */
#define MRT_BUF_CROSS_K 1     /* layer: (rows, heads, enc_len, d_kv)            */
#define MRT_BUF_CROSS_V 2
#define MRT_BUF_TEMPORAL_K 3  /* layer: (rows, heads, max_frames, d_kv) ring    */
#define MRT_BUF_TEMPORAL_V 4
#define MRT_BUF_DEPTH_K 5     /* layer: (rows, heads, rvq_depth, d_kv) ring     */
#define MRT_BUF_DEPTH_V 6
#define MRT_BUF_ENC_TOKENS 7  /* (rows, enc_len) int32 ids of the last encode; read-only */
int mrt_df_state_buffer_bytes(mrt_df_state* st, int which, size_t* bytes);
int mrt_df_state_read(mrt_df_state* st, int which, int layer, void* dst, size_t bytes);
int mrt_df_state_write(mrt_df_state* st, int which, int layer, const void* src, size_t bytes);
/* Declare how many ring slots hold valid K/V (kind 0: temporal, 1: depth), e.g.
 * after mrt_df_state_write for a step micro-benchmark at a given cache length. */
int mrt_df_state_set_cache_length(mrt_df_state* st, int kind, int length);

/* ---- Streaming: the token half of System::generate_chunk on the device ----
 *
 * System::generate_chunk (system.cpp:177-370) without the codec: the RVQ
 * context (SystemState::context_tokens, system.h:124-130) stays in device
 * memory.  Per chunk, on the stream's HIP stream: the encoder inputs are
 * built from the context and the style (build_encoder_inputs_host,
 * system.cpp:62-95), the encoder and the 50x16 decode run, the LLM ids are
 * turned into RVQ codes (llm_to_rvq safe mode, rvq.cpp:112-132) and rolled
 * into the context (system.cpp:315-333).  Only the chunk's ids leave the
 * device. */

/* The SystemConfig fields the token half reads (system.h:44-83). */
typedef struct mrt_stream_config {
  int32_t chunk_frames;            /* 50  chunk_length_frames */
  int32_t context_frames;          /* 250 context_length_frames */
  int32_t codebook_size;           /* 1024 codec_rvq_codebook_size */
  int32_t encoder_codec_rvq_depth; /* 4 */
  int32_t encoder_style_rvq_depth; /* 6 */
  int32_t decoder_codec_rvq_depth; /* 16 (= the model's rvq_depth) */
  int32_t mask_token;              /* 1  vocab_mask_token */
  int32_t codec_offset;            /* 2  vocab_codec_offset */
  int32_t crossfade_frames;        /* 1  crossfade_length_frames (0.04 s x 25 Hz) */
  int32_t samples_per_frame;       /* 1920 codec_sample_rate / codec_frame_rate */
} mrt_stream_config;

/* GenerateChunkOptions (system.h:86-121). */
typedef struct mrt_chunk_opts {
  float temperature;        /* 1.1 */
  int32_t top_k;            /* 40 */
  float guidance_weight;    /* 5.0 */
  int32_t has_seed;         /* 0: the stream picks base + chunk_index from a random base */
  uint64_t seed;
  int32_t pipeline_encoder; /* enqueue the next chunk's encoder before returning */
  int32_t use_graph;        /* replay the decode loop from a captured hipGraph */
  const int32_t* teacher;   /* optional host (chunk_frames, levels) ids fed back instead of draws */
  int32_t speculative;      /* speculative depth decoding, drafts = the previous chunk's tokens:
                               0 off, 1 on, 2 adaptive (a chunk speculates its first 2 frames only;
                               when >= 1/4 of those levels came from the verification pass, whole
                               chunks speculate while that holds; after a miss, 4 chunks plain
                               before the next probe, doubling per further miss up to 64) */
} mrt_chunk_opts;

typedef struct mrt_df_stream mrt_df_stream;
typedef struct mrt_codec mrt_codec; /* the codec decode handle (declared below) */

/* SystemConfig defaults (system.h:44-83) / GenerateChunkOptions defaults. */
void mrt_stream_config_default(mrt_stream_config* cfg);
void mrt_chunk_opts_default(mrt_chunk_opts* opts);

/* System::empty_state (system.cpp:165-176): every context slot empty (-1),
 * chunk index 0.  Owns a state with rows = 2, max_frames = chunk_frames and
 * enc_len = context_frames * encoder_codec_rvq_depth + encoder_style_rvq_depth. */
int mrt_df_stream_create(mrt_df* h, const mrt_stream_config* cfg, mrt_df_stream** out);
void mrt_df_stream_destroy(mrt_df_stream* s);

/* System::generate_chunk (system.cpp:177-370), token half.  style: host
 * (encoder_style_rvq_depth) style-vocab ids or NULL (masked), as
 * style_tokens_lm.  llm_out / rvq_out: host (chunk_frames, levels) or NULL:
 * the chunk's LLM ids (SystemState::last_frame_tokens_llm) and RVQ codes.
 * A decoded id at the wrong level fails with MRT_ERR_INVALID and
 * "llm_to_rvq: token levels do not match expected RVQ structure" (the
 * reference's std::invalid_argument); the context and chunk index are then
 * unchanged.  With pipeline_encoder the next chunk's encoder is enqueued
 * before returning and reused by the next call if its style is the same
 * (system.cpp:218-232, 334-370). */
int mrt_df_stream_generate_chunk(mrt_df_stream* s, const int32_t* style, const mrt_chunk_opts* opts,
                                 int32_t* llm_out, int32_t* rvq_out);

/* The whole System::generate_chunk (system.cpp:177-440) on the device: the
 * token half as mrt_df_stream_generate_chunk, then the codec decode of
 * [crossfade_frames context frames before the chunk (ids clamped at 0; zeros
 * on chunk 0), the chunk's codes] (system.cpp:294-313, 373-390) on the
 * attached codec's stream -- overlapping the pipelined encoder of the next
 * chunk -- and the equal-power crossfade against the previous chunk's tail
 * (system.cpp:395-440).  audio_out: host (chunk_frames * samples_per_frame,
 * 2) float32, L/R interleaved (GenerateResult::waveform).  The crossfade
 * applies when the previous call of the stream also produced audio. */
int mrt_df_stream_generate_chunk_audio(mrt_df_stream* s, const int32_t* style, const mrt_chunk_opts* opts,
                                       int32_t* llm_out, int32_t* rvq_out, float* audio_out);
/* compile_for_inference for a stream (system.cpp:130 calls it once after
 * loading): mrt_df_state_compile of the stream's state with the decode
 * options of a chunk under `opts`, after building the encoder inputs of the
 * current context (masked style) and running the encoder, unless a pipelined
 * encoder output is held.  The context and chunk index are unchanged. */
int mrt_df_stream_compile(mrt_df_stream* s, const mrt_chunk_opts* opts);

/* Attach a codec (not owned; NULL detaches) to a stream.  Its rvq_levels and
 * codebook_size must equal the stream's and its max_frames must be at least
 * chunk_frames + crossfade_frames.  The codec must outlive the stream or be
 * detached first; its launch plan for the chunk size is built here. */
int mrt_df_stream_attach_codec(mrt_df_stream* s, mrt_codec* c);

/* SystemState::context_tokens and chunk_index in and out: host
 * (context_frames, levels) int32, -1 = empty.  set_context drops a
 * pipelined encoder output. */
int mrt_df_stream_set_context(mrt_df_stream* s, const int32_t* context, int64_t chunk_index);
int mrt_df_stream_get_context(mrt_df_stream* s, int32_t* context, int64_t* chunk_index);

/* The stream's decode state, for the instrumentation and buffer calls above
 * (mrt_df_state_decode_time, mrt_df_state_read).  Owned by the stream:
 * valid until mrt_df_stream_destroy; mrt_df_state_destroy ignores it. */
int mrt_df_stream_state(mrt_df_stream* s, mrt_df_state** st);

/* ---- Batched independent streams ----------------------------------------------
 *
 * No counterpart in the reference, whose generate_tokens decodes one stream
 * (decode.cpp:239-573); this is the same loop for `streams` independent
 * streams (each its own encoder tokens, seed and KV caches) run together as
 * 2 * streams activation rows, so the projections become skinny GEMMs on the
 * matrix cores.  Per stream the semantics are those of
 * mrt_df_generate_tokens.  bf16 models only; streams <= 32. */
typedef struct mrt_df_batch mrt_df_batch;

/* KV rings for `max_frames` temporal steps and rvq_depth depth steps per
 * stream; encoder length enc_len (<= max_encoder_length). */
int mrt_df_batch_create(mrt_df* h, int streams, int max_frames, int enc_len, mrt_df_batch** out);
void mrt_df_batch_destroy(mrt_df_batch* b);
/* Depthformer::encode (model.cpp:226-241) of every stream: tokens
 * (2 * streams, enc_len) host int32, rows 2s and 2s + 1 = stream s's CFG
 * pair; then the cross K/V of every temporal layer. */
int mrt_df_batch_encode(mrt_df_batch* b, const int32_t* tokens);
/* One chunk of every stream: enc_tokens as mrt_df_batch_encode (NULL: reuse
 * the last encode); seeds (streams) host, stream s draws with seeds[s];
 * opts->teacher, when set, is host (streams, num_frames, rvq_depth);
 * opts->record_slices (device (F, L, 2 * streams, codebook)) and
 * opts->record_temporal (device (F, 2 * streams, d_model)) are honoured,
 * record_drawn / record_frame_mean must be NULL.  out_tokens: host
 * (streams, num_frames, rvq_depth) LLM ids. */
int mrt_df_batch_generate_tokens(mrt_df_batch* b, const int32_t* enc_tokens, const mrt_gen_opts* opts,
                                 const uint64_t* seeds, int32_t* out_tokens);
/* The batch's hipStream_t (all its work is ordered on it). */
int mrt_df_batch_stream(mrt_df_batch* b, void** hip_stream);
/* GPU ms of the last generate call's decode section (HIP events on the
 * batch's stream); instrumentation, as mrt_df_state_decode_time. */
int mrt_df_batch_decode_time(mrt_df_batch* b, float* ms);
/* Device copy of the encoder output (2 * streams, enc_len, d_model) (model
 * dtype) into dst, for parity checks. */
int mrt_df_batch_read_enc_out(mrt_df_batch* b, void* dst, size_t bytes);

/* ------------------------------------------------------------------------
 * Codec decode: the audio half of System::generate_chunk (system.cpp:
 * 373-390): rvq_dequantization (rvq.cpp:68-88) with the SpectroStream
 * codebooks, SpectroStreamDecoder::operator() (spectrostream.cpp:365-432)
 * and istft_postprocess (spectrostream.cpp:593-681), all in fp32 as the
 * reference runs them (system.cpp:118-119).
 * ------------------------------------------------------------------------ */
typedef struct {
  int32_t embedding_dim;   /* 256: SpectroStreamDecoder::kEmbeddingDim */
  int32_t proj_channels;   /* 2560: input_proj 256 -> 2560 -> 2560 (spectrostream.cpp:356-362) */
  int32_t unfold;          /* 5: unfold_width factor (2560 = 5 x 512) */
  int32_t block_in[7];     /* decoder block channels (spectrostream.cpp:328-338); the */
  int32_t block_out[7];    /*   strides, kernels and crops are the reference's */
  int32_t rvq_levels;      /* 16: codebooks summed per frame */
  int32_t codebook_size;   /* 1024 */
  int32_t max_frames;      /* largest decode the handle serves (51 = 1 crossfade + 50) */
} mrt_codec_config;

#define MRT_CODEC_BUF_EMB 0         /* (frames + 1, 256) dequantised embeddings + the zero pad frame */
#define MRT_CODEC_BUF_INPUT_CONV 1  /* (1, frames + 1, 5, 512) after input_proj + input_conv */
#define MRT_CODEC_BUF_BLOCK0 2      /* 2..8: decoder block i output, (2, H, W, C) after block 0's stereo split */
#define MRT_CODEC_BUF_SPEC 9        /* (2, 4 frames, 480, 2): stereo half s, (real, imag) -- the decoder
                                       output before the (B, H, 480, 4) interleave */
#define MRT_CODEC_BUF_FRAMES 10     /* (2 x 4 frames, 960) windowed iSTFT frames */

/* The reference's decoder configuration (SpectroStreamDecoder, the decoder
 * block table and SystemConfig's 1 crossfade frame + 50 chunk frames). */
void mrt_codec_config_default(mrt_codec_config* cfg);
/* SpectroStreamDecoder(bundle, float32) (spectrostream.cpp:356-362) from
 * spectrostream_decoder.safetensors plus the "codebooks" tensor (K, C, 256)
 * of spectrostream_codebooks.safetensors (weights.cpp:80-83; system.cpp:
 * 105-119).  Conv weights (out, in, kH, kW), transposed-conv weights (in,
 * out, kH, kW), as stored. */
int mrt_codec_create(const char* decoder_path, const char* codebooks_path, const mrt_codec_config* cfg, int device,
                     mrt_codec** out);
/* The same from caller-owned fp32 host arrays (decoder keys and "codebooks"). */
int mrt_codec_create_from_tensors(int n, const char* const* names, const float* const* data,
                                  const int64_t* const* shapes, const int32_t* ndims, const mrt_codec_config* cfg,
                                  int device, mrt_codec** out);
void mrt_codec_destroy(mrt_codec* c);
/* system.cpp:373-390: rvq_tokens host (frames, rvq_levels) int32 in [0,
 * codebook_size) -> audio host (frames * 1920, 2) float32, L/R interleaved
 * (istft_postprocess with target length frames * 48000 / 25).  Ids outside
 * the codebook return MRT_ERR_INVALID before any device work. */
int mrt_codec_decode(mrt_codec* c, const int32_t* rvq_tokens, int frames, float* audio);
/* The same on device pointers, enqueued on the codec's stream without a host
 * sync (ids outside the codebook are read as 0). */
int mrt_codec_decode_device(mrt_codec* c, const int32_t* rvq_tokens_dev, int frames, float* audio_dev);
/* The codec's hipStream_t, a wait for its work, and the GPU ms of the last
 * decode (HIP events on its stream). */
int mrt_codec_stream(mrt_codec* c, void** hip_stream);
int mrt_codec_sync(mrt_codec* c);
int mrt_codec_decode_time(mrt_codec* c, float* ms);
/* Copy of an intermediate of the last decode (MRT_CODEC_BUF_*); bytes must
 * equal its size at that decode's frame count. */
int mrt_codec_read(mrt_codec* c, int which, void* dst, size_t bytes);

/* ------------------------------------------------------------------------
 * MusicCoCa text path and style tokens (StyleModel, style_model.cpp:76-121;
 * MusicCoCaEncoder::embed_text, musiccoca.cpp:272-294; rvq_quantization,
 * rvq.cpp:24-62), fp32 as the reference's StyleModel default.  The
 * SentencePiece tokenizer stays with the caller: ids come in laid out as
 * StyleModel::tokenize_text_ids (style_model.cpp:52-74) does -- BOS (1),
 * the lower-cased prompt's ids, zeros; padding 1.0 on the padded slots.
 * ------------------------------------------------------------------------ */
typedef struct mrt_coca mrt_coca;

typedef struct {
  int32_t d_model;       /* 768  MusicCoCaConfig (musiccoca.h:151-162) */
  int32_t num_heads;     /* 12 */
  int32_t d_head;        /* 64 */
  int32_t d_ff;          /* 3072 */
  int32_t num_layers;    /* 12 */
  int32_t pooler_d_head; /* 256 */
  int32_t vocab_size;    /* 64000 */
  int32_t max_text_len;  /* 128  StyleModel::kMaxTextLength */
  int32_t rvq_depth;     /* 12   StyleModel::kRVQDepth */
  int32_t codebook_size; /* 1024 StyleModel::kRVQCodebookSize */
} mrt_coca_config;

#define MRT_COCA_BUF_EMBEDDING 0 /* (d_model) the last embedding; 1 + i: text layer i's output (max_text_len, d_model) */

void mrt_coca_config_default(mrt_coca_config* cfg);
/* StyleModel(encoder_bundle, codebooks_bundle) (style_model.cpp:37-50): the
 * text-path keys of the MusicCoCa bundle (Linear weights (out, in)) and the
 * "codebooks" tensor (K >= rvq_depth, codebook_size, d_model). */
int mrt_coca_create(const char* encoder_path, const char* codebooks_path, const mrt_coca_config* cfg, int device,
                    mrt_coca** out);
int mrt_coca_create_from_tensors(int n, const char* const* names, const float* const* data,
                                 const int64_t* const* shapes, const int32_t* ndims, const mrt_coca_config* cfg,
                                 int device, mrt_coca** out);
void mrt_coca_destroy(mrt_coca* h);
/* MusicCoCaEncoder::embed_text of one prompt: ids (max_text_len) int32 and
 * padding (max_text_len) float, host -> embedding (d_model) float, host.
 * The second call on a handle captures the launch sequence into a HIP graph
 * that later calls replay (same results as the direct launches). */
int mrt_coca_embed_text(mrt_coca* h, const int32_t* ids, const float* padding, float* embedding);
/* StyleModel::tokenize: embedding host (d_model), or NULL for the last
 * mrt_coca_embed_text result -> tokens (rvq_depth) int32, host. */
int mrt_coca_tokenize(mrt_coca* h, const float* embedding, int32_t* tokens);
/* StyleModel::style_tokens_lm: embed, tokenize, keep the first style_depth
 * levels, then offset + level * codebook + token (rvq_to_llm, rvq.cpp:98-103). */
int mrt_coca_style_tokens_lm(mrt_coca* h, const int32_t* ids, const float* padding, int style_depth,
                             int style_codebook_size, int vocab_style_offset, int32_t* out);
/* GPU ms of the last embed_text (HIP events on the handle's stream). */
int mrt_coca_embed_time(mrt_coca* h, float* ms);
/* Copy of an intermediate of the last embed_text (MRT_COCA_BUF_*); bytes must match. */
int mrt_coca_read(mrt_coca* h, int which, void* dst, size_t bytes);

#ifdef __cplusplus
}
#endif

#endif /* MRT_DF_H_ */
