// Batched independent streams (see batch.hpp).  The decode loop is the
// per-layer loop of generate_tokens (decode.cpp:339-486) with R = 2B rows in
// every kernel: skinny MFMA GEMMs for the projections, the ring / cross
// attention and sampling kernels over all rows, the residual stream updated
// in place.  With use_graph, one frame (temporal step, 16 depth steps and
// draws) is captured once, reading its frame index from a device counter, and
// replayed for every frame.
#include "batch.hpp"

#include <algorithm>
#include <cstring>

#include "kernels.hpp"

namespace mrt {

void* Batch::dalloc(size_t bytes) {
  void* d = nullptr;
  MRT_HIP_CHECK(hipMalloc(&d, std::max<size_t>(bytes, 256)));
  allocs_.push_back(d);
  return d;
}

Batch::Batch(Model& model, int streams, int max_frames, int enc_len)
    : m(model), B(streams), R(2 * streams), F(max_frames), S(enc_len) {
  const Config& c = m.cfg;
  MRT_REQUIRE(m.dt == DType::BF16, "batched streams run in bf16 (load the model with dtype bf16)");
  MRT_REQUIRE(B >= 1 && R <= kBatchRows, "streams must be in [1, 32]");
  MRT_REQUIRE(F >= 1 && F <= 1024, "max_frames must be in [1, 1024]");
  MRT_REQUIRE(S >= 1 && S <= c.max_encoder_length, "enc_len must be in [1, max_encoder_length]");
  MRT_REQUIRE(c.d_model % 32 == 0 && c.hd() % 32 == 0 && c.d_ff % 32 == 0,
              "batched streams need d_model, heads * 64 and d_ff multiples of 32");
  MRT_HIP_CHECK(hipSetDevice(m.device));
  MRT_HIP_CHECK(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking));
  const size_t D = c.d_model, HD = c.hd(), FF = c.d_ff, H = c.num_heads, L = c.rvq_depth, e = 2;
  const size_t M = static_cast<size_t>(R) * S;
  enc_.rows = R;
  enc_.S = S;
  enc_.tok = static_cast<int*>(dalloc(M * 4));
  enc_.ex = dalloc(M * D * e);
  enc_.exn = dalloc(M * D * e);
  enc_.eqkv = dalloc(M * 3 * HD * e);
  enc_.eattn = dalloc(M * HD * e);
  enc_.effh = dalloc(M * FF * e);
  enc_.enc_out = dalloc(M * D * e);
  enc_.cross = dalloc(static_cast<size_t>(c.num_temporal_layers) * 2 * R * H * S * 64 * e);
  tkv_ = dalloc(static_cast<size_t>(c.num_temporal_layers) * 2 * R * H * F * 64 * e);
  dkv_ = dalloc(static_cast<size_t>(c.num_depth_layers) * 2 * R * H * L * 64 * e);
  t_in_ = dalloc(R * D * e);
  d_in_ = dalloc(R * D * e);
  xn_ = dalloc(R * std::max(D, FF) * e);
  ssq_ = static_cast<float*>(dalloc(static_cast<size_t>(R) * (D / 16) * 4));
  q_ = dalloc(R * HD * e);
  att_ = dalloc(R * HD * e);
  ffh_ = dalloc(R * FF * e);
  fsum_ = dalloc(R * D * e);
  logits_ = static_cast<float*>(dalloc(static_cast<size_t>(R) * 1024 * 4));
  noise_ = static_cast<float*>(dalloc(static_cast<size_t>(B) * F * L * 1024 * 4));
  d_tokens_ = static_cast<int*>(dalloc(static_cast<size_t>(B) * F * L * 4));
  d_teacher_ = static_cast<int*>(dalloc(static_cast<size_t>(B) * F * L * 4));
  d_frame_ = static_cast<int*>(dalloc(4));
  d_seeds_ = static_cast<uint64_t*>(dalloc(static_cast<size_t>(B) * 8));
  h_pinned_n_ = std::max<size_t>(M, static_cast<size_t>(B) * F * L + 2 * B);
  MRT_HIP_CHECK(hipHostMalloc(reinterpret_cast<void**>(&h_pinned_), h_pinned_n_ * 4, hipHostMallocDefault));
  MRT_HIP_CHECK(hipEventCreate(&ev_[0]));
  MRT_HIP_CHECK(hipEventCreate(&ev_[1]));
}

Batch::~Batch() {
  (void)hipSetDevice(m.device);
  if (stream) (void)hipStreamSynchronize(stream);
  if (graph_exec_) (void)hipGraphExecDestroy(graph_exec_);
  if (graph_) (void)hipGraphDestroy(graph_);
  for (hipEvent_t e : ev_)
    if (e) (void)hipEventDestroy(e);
  for (void* p : allocs_) (void)hipFree(p);
  if (h_pinned_) (void)hipHostFree(h_pinned_);
  if (stream) (void)hipStreamDestroy(stream);
}

char* Batch::ring(void* base, int layer, int kv, int len) const {
  const size_t n = static_cast<size_t>(R) * m.cfg.num_heads * len * 64 * 2;
  return static_cast<char*>(base) + (2 * static_cast<size_t>(layer) + kv) * n;
}

void Batch::encode(const int32_t* tokens_host) {
  const size_t M = static_cast<size_t>(R) * S;
  for (size_t i = 0; i < M; ++i)
    MRT_REQUIRE(tokens_host[i] >= 0 && tokens_host[i] < m.cfg.vocab_size, "encode: token id out of range");
  MRT_HIP_CHECK(hipSetDevice(m.device));
  MRT_HIP_CHECK(hipStreamSynchronize(stream));  // staging reuse
  std::memcpy(h_pinned_, tokens_host, M * 4);
  MRT_HIP_CHECK(hipMemcpyAsync(enc_.tok, h_pinned_, M * 4, hipMemcpyHostToDevice, stream));
  encode_device();
}

void Batch::encode_device() {
  MRT_HIP_CHECK(hipSetDevice(m.device));
  run_encoder(m, enc_, stream);
  encoded_ = true;
}

// Temporal step of every row in place on t_in_ (model.cpp:493-513 per row):
// ring slot f, or *fptr when non-null.
void Batch::temporal_stack(int f, const int* fptr) {
  const Config& c = m.cfg;
  const int D = c.d_model, HD = c.hd(), FF = c.d_ff, H = c.num_heads;
  for (int i = 0; i < c.num_temporal_layers; ++i) {
    const DecoderLayerW& W = m.tmp[i];
    char *tk = ring(tkv_, i, 0, F), *tv = ring(tkv_, i, 1, F);
    // layer 0's input is the frame mean (no row partials): a plain norm pass
    if (i == 0) {
      rmsnorm_rows(DType::BF16, t_in_, W.norm_sa, 1e-6f, R, D, xn_, stream);
      bgemm_qkv(xn_, R, D, W.wqkv, HD, q_, tk, tv, H, F, f, fptr, stream);
    } else {
      bgemm_qkv(t_in_, R, D, W.wqkv, HD, q_, tk, tv, H, F, f, fptr, stream, norm(W.norm_sa));
    }
    self_attn_at(DType::BF16, R, q_, tk, tv, H, F, f + 1, f, fptr, m.tbias, m.tbuckets, att_, stream);
    bgemm_resid(att_, R, HD, W.wo, D, t_in_, D, stream, ssq_);
    bgemm_store(t_in_, R, D, W.wq_c, HD, q_, HD, stream, norm(W.norm_ca));
    cross_attn_rows(q_, ring(enc_.cross, i, 0, S), ring(enc_.cross, i, 1, S), R, H, S, att_, stream);
    bgemm_resid(att_, R, HD, W.wo_c, D, t_in_, D, stream, ssq_);
    bgemm_geglu(t_in_, R, D, W.w01, FF, ffh_, FF, stream, norm(W.norm_ff));
    bgemm_resid(ffh_, R, FF, W.wo2, D, t_in_, D, stream, ssq_);
  }
}

// Depth step l of every row in place on x (model.cpp:638-651 per row).
// x_partials: the row partials of x are those the last bgemm_resid left
// (the temporal step's output), else layer 0 normalises in its own pass.
// qkv_fed: layer 0's q and ring slot l were written by the previous level's
// draw from the q/k/v table (x = emb(token), a function of the token alone).
void Batch::depth_stack(void* x, int l, bool x_partials, bool qkv_fed) {
  const Config& c = m.cfg;
  const int D = c.d_model, HD = c.hd(), FF = c.d_ff, H = c.num_heads, L = c.rvq_depth;
  for (int i = 0; i < c.num_depth_layers; ++i) {
    const DecoderLayerW& W = m.dep[i];
    char *dk = ring(dkv_, i, 0, L), *dv = ring(dkv_, i, 1, L);
    if (i == 0 && qkv_fed) {
      // nothing to compute: q / k / v are in place
    } else if (i == 0 && !x_partials) {
      rmsnorm_rows(DType::BF16, x, W.norm_sa, 1e-6f, R, D, xn_, stream);
      bgemm_qkv(xn_, R, D, W.wqkv, HD, q_, dk, dv, H, L, l, nullptr, stream);
    } else {
      bgemm_qkv(x, R, D, W.wqkv, HD, q_, dk, dv, H, L, l, nullptr, stream, norm(W.norm_sa));
    }
    self_attn_at(DType::BF16, R, q_, dk, dv, H, L, l + 1, l, nullptr, m.dbias, m.dbuckets, att_, stream);
    bgemm_resid(att_, R, HD, W.wo, D, x, D, stream, ssq_);
    bgemm_geglu(x, R, D, W.w01, FF, ffh_, FF, stream, norm(W.norm_ff));
    bgemm_resid(ffh_, R, FF, W.wo2, D, x, D, stream, ssq_);
  }
}

// One frame of every stream (decode.cpp:339-486): the temporal step on the
// previous frame's mean, then per level the depth step, decoder_norm, the
// level's lm_head rows and the draws, which feed emb(token) to the next level
// and at the last level leave the frame mean in t_in_.  dynamic: the frame
// index comes from d_frame_ (graph replay), which the frame then advances.
void Batch::enqueue_frame(const GenOpts& o, int f, bool dynamic) {
  const Config& c = m.cfg;
  const int D = c.d_model, L = o.rvq_depth, C = o.codebook;
  const int* fptr = dynamic ? d_frame_ : nullptr;
  const size_t row_bytes = static_cast<size_t>(R) * D * 2;
  SampleParams sp{o.guidance_weight, o.temperature, o.top_k, C, o.codec_offset, L, d_seeds_, noise_, F};
  QkvFeed feed;
  if (qkv_tab_ != nullptr) {
    feed.table = qkv_tab_;
    feed.q = q_;
    feed.kc = ring(dkv_, 0, 0, c.rvq_depth);
    feed.vc = ring(dkv_, 0, 1, c.rvq_depth);
    feed.HD = c.hd();
    feed.H = c.num_heads;
    feed.Lmax = c.rvq_depth;
    feed.offset = o.codec_offset;
    feed.rows = (L - 1) * C;
  }
  temporal_stack(f, fptr);
  if (o.record_temporal) copy_dev(static_cast<char*>(o.record_temporal) + f * row_bytes, t_in_, row_bytes, stream);
  for (int l = 0; l < L; ++l) {
    void* x = l == 0 ? t_in_ : d_in_;
    depth_stack(x, l, l == 0 && c.num_temporal_layers > 0, l > 0 && qkv_tab_ != nullptr);
    const char* head = static_cast<const char*>(m.lm_head) + static_cast<size_t>(o.codec_offset + C * l) * D * 2;
    if (c.num_depth_layers > 0) {
      bgemm_f32(x, R, D, head, C, logits_, C, stream, norm(m.dec_norm));
    } else {
      rmsnorm_rows(DType::BF16, x, m.dec_norm, 1e-6f, R, D, xn_, stream);
      bgemm_f32(xn_, R, D, head, C, logits_, C, stream);
    }
    if (o.record_slices)
      copy_dev(o.record_slices + (static_cast<size_t>(f) * L + l) * R * C, logits_, static_cast<size_t>(R) * C * 4,
               stream);
    sample_levels(DType::BF16, B, logits_, sp, f, fptr, l, dynamic ? l : f * L + l, F * L,
                  o.teacher ? d_teacher_ : nullptr, d_tokens_, nullptr, m.emb, D, d_in_, fsum_, t_in_, stream,
                  qkv_tab_ != nullptr ? &feed : nullptr);
  }
  if (dynamic) advance_counter(d_frame_, stream);
}

void Batch::generate(const int32_t* enc_tokens_host, const GenOpts& o, const uint64_t* seeds, int32_t* out_host) {
  const Config& c = m.cfg;
  MRT_REQUIRE(o.num_frames >= 1 && o.num_frames <= F, "generate: num_frames exceeds the batch's max_frames");
  MRT_REQUIRE(o.rvq_depth == c.rvq_depth, "generate: rvq_depth must equal the model's rvq_depth");
  MRT_REQUIRE(o.codebook >= 1 && o.codebook <= 1024, "generate: codebook_size must be in [1, 1024]");
  MRT_REQUIRE(o.codec_offset >= 0 && o.codec_offset + o.codebook * o.rvq_depth <= c.vocab_size,
              "generate: codec levels exceed the vocabulary");
  MRT_REQUIRE(o.temperature >= 0.0f, "generate: temperature must be >= 0");
  MRT_REQUIRE(seeds != nullptr, "generate: seeds are required (one per stream)");
  MRT_HIP_CHECK(hipSetDevice(m.device));
  if (enc_tokens_host) encode(enc_tokens_host);
  if (!encoded_) throw Error(2, "generate: no encoder output (pass enc_tokens or call encode)");
  const int L = o.rvq_depth;
  const size_t nt = static_cast<size_t>(B) * F * L;
  MRT_HIP_CHECK(hipStreamSynchronize(stream));  // staging reuse
  std::memcpy(h_pinned_, seeds, static_cast<size_t>(B) * 8);
  MRT_HIP_CHECK(hipMemcpyAsync(d_seeds_, h_pinned_, static_cast<size_t>(B) * 8, hipMemcpyHostToDevice, stream));
  if (o.teacher) {
    // host (B, num_frames, L) -> device (B, F, L)
    const size_t per = static_cast<size_t>(o.num_frames) * L;
    for (size_t i = 0; i < static_cast<size_t>(B) * per; ++i)
      MRT_REQUIRE(o.teacher[i] >= 0 && o.teacher[i] < c.vocab_size, "generate: teacher id out of range");
    int32_t* t = h_pinned_ + 2 * B;
    std::fill(t, t + nt, 0);
    for (int b = 0; b < B; ++b) std::memcpy(t + static_cast<size_t>(b) * F * L, o.teacher + b * per, per * 4);
    MRT_HIP_CHECK(hipMemcpyAsync(d_teacher_, t, nt * 4, hipMemcpyHostToDevice, stream));
  }
  MRT_HIP_CHECK(hipStreamSynchronize(stream));
  // Depth layer 0 of levels 1.. reads the model's q/k/v table row of the fed
  // token (built once per codec levels, before any capture) when every fed
  // token lies in it: drawn tokens always do, teacher tokens are checked.
  bool in_table = c.num_depth_layers > 0 && L >= 2;
  if (o.teacher != nullptr) {
    const size_t per = static_cast<size_t>(o.num_frames) * L;
    for (int b = 0; b < B && in_table; ++b)
      for (int f = 0; f < o.num_frames && in_table; ++f)
        for (int l = 0; l + 1 < L; ++l) {
          const int id = o.teacher[b * per + static_cast<size_t>(f) * L + l];
          if (id < o.codec_offset + l * o.codebook || id >= o.codec_offset + (l + 1) * o.codebook) {
            in_table = false;
            break;
          }
        }
  }
  qkv_tab_ = in_table ? m.depth_qkv_table(o.codebook, o.codec_offset, stream) : nullptr;

  const bool graph = o.use_graph && !o.record_slices && !o.record_temporal;
  MRT_HIP_CHECK(hipEventRecord(ev_[0], stream));
  // The noise of every draw, tabulated once (the sampler reads it instead of
  // running Philox per candidate); then frame 0 feeds emb(PAD = 0) on every
  // row (decode.cpp:339-341, 366-368).
  if (o.temperature != 0.0f) gumbel_tables(d_seeds_, B, F, L, o.codebook, noise_, stream);
  embed_fill(DType::BF16, m.emb, c.d_model, 0, R, t_in_, stream);
  if (graph) {
    const std::vector<double> key = {(double)L, (double)o.temperature, (double)o.top_k, (double)o.guidance_weight,
                                     (double)o.codebook, (double)o.codec_offset, o.teacher ? 1.0 : 0.0,
                                     qkv_tab_ != nullptr ? 1.0 : 0.0};
    if (!graph_exec_ || key != graph_key_) {
      if (graph_exec_) (void)hipGraphExecDestroy(graph_exec_);
      if (graph_) (void)hipGraphDestroy(graph_);
      graph_exec_ = nullptr;
      graph_ = nullptr;
      MRT_HIP_CHECK(hipStreamSynchronize(stream));  // capture starts on an idle stream
      MRT_HIP_CHECK(hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal));
      try {
        enqueue_frame(o, 0, true);
      } catch (...) {
        hipGraph_t g = nullptr;
        (void)hipStreamEndCapture(stream, &g);
        if (g) (void)hipGraphDestroy(g);
        throw;
      }
      MRT_HIP_CHECK(hipStreamEndCapture(stream, &graph_));
      MRT_HIP_CHECK(hipGraphInstantiate(&graph_exec_, graph_, nullptr, nullptr, 0));
      graph_key_ = key;
    }
    set_counter(d_frame_, 0, stream);
    for (int f = 0; f < o.num_frames; ++f) MRT_HIP_CHECK(hipGraphLaunch(graph_exec_, stream));
  } else {
    for (int f = 0; f < o.num_frames; ++f) enqueue_frame(o, f, false);
  }
  MRT_HIP_CHECK(hipEventRecord(ev_[1], stream));
  timed_ = true;
  MRT_HIP_CHECK(hipMemcpyAsync(h_pinned_, d_tokens_, nt * 4, hipMemcpyDeviceToHost, stream));
  MRT_HIP_CHECK(hipStreamSynchronize(stream));
  const size_t per = static_cast<size_t>(o.num_frames) * L;
  for (int b = 0; b < B; ++b) std::memcpy(out_host + b * per, h_pinned_ + static_cast<size_t>(b) * F * L, per * 4);
}

float Batch::last_decode_ms() const {
  if (!timed_) throw Error(1, "decode time: no generate call on this batch yet");
  MRT_HIP_CHECK(hipEventSynchronize(ev_[1]));
  float ms = 0.f;
  MRT_HIP_CHECK(hipEventElapsedTime(&ms, ev_[0], ev_[1]));
  return ms;
}

}  // namespace mrt
