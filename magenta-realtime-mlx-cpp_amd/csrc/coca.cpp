// MusicCoCa text path host side: weight packing (Q/K/V fused, the pooler's
// K/V fused), the fixed GEMM plan of one prompt (max_text_len rows) and the
// launch sequence of MusicCoCaEncoder::embed_text (musiccoca.cpp:272-294) and
// StyleModel::tokenize (style_model.cpp:88-104).
#include "coca.hpp"

#include <algorithm>
#include <cmath>
#include <string>

namespace mrt {

namespace {

int round_up(int v, int m) { return (v + m - 1) / m * m; }

void check_shape(const HostTensor& t, const std::string& name, std::vector<int64_t> want) {
  if (t.shape != want) throw Error(1, "musiccoca: tensor " + name + " has an unexpected shape");
}

}  // namespace

float* Coca::dalloc(size_t floats) {
  void* d = nullptr;
  MRT_HIP_CHECK(hipMalloc(&d, std::max<size_t>(floats * 4, 256)));
  allocs_.push_back(d);
  return static_cast<float*>(d);
}

// Linear (musiccoca.cpp:85-98), stored (out, in): several stored matrices
// with the same input width stacked along the output axis, packed (in,
// out_pad) for the GEMM, biases concatenated.
Coca::Lin Coca::pack(const TensorSource& w, const std::vector<std::string>& names, int in) {
  Lin l;
  l.in = in;
  for (const auto& n : names) l.out += static_cast<int>(w.tensor(n + ".weight").shape[0]);
  l.out_pad = round_up(l.out, 64);
  std::vector<float> h(static_cast<size_t>(in) * l.out_pad, 0.f), hb(l.out);
  int o0 = 0;
  for (const auto& n : names) {
    const HostTensor& t = w.tensor(n + ".weight");
    const HostTensor& b = w.tensor(n + ".bias");
    const int o = static_cast<int>(t.shape[0]);
    for (int r = 0; r < o; ++r) {
      for (int c = 0; c < in; ++c) h[static_cast<size_t>(c) * l.out_pad + o0 + r] = t.data[static_cast<size_t>(r) * in + c];
      hb[o0 + r] = b.data[r];
    }
    o0 += o;
  }
  l.w = dalloc(h.size());
  MRT_HIP_CHECK(hipMemcpy(l.w, h.data(), h.size() * 4, hipMemcpyHostToDevice));
  l.b = dalloc(l.out);
  MRT_HIP_CHECK(hipMemcpy(l.b, hb.data(), hb.size() * 4, hipMemcpyHostToDevice));
  return l;
}

Coca::Coca(const TensorSource& w, const TensorSource& cbs, const CocaConfig& c, int dev) : cfg(c), device(dev) {
  const int D = c.d_model, HD = c.num_heads * c.d_head, PD = c.num_heads * c.pooler_d_head, F = c.d_ff;
  const int L = c.max_text_len;
  MRT_REQUIRE(D >= 16 && D % 16 == 0 && F % 16 == 0 && HD % 16 == 0 && PD % 16 == 0,
              "musiccoca: widths must be multiples of 16");
  MRT_REQUIRE(L >= 1 && L <= 256, "musiccoca: max_text_len must be in [1, 256]");
  MRT_REQUIRE(c.d_head <= 256 && c.pooler_d_head <= 256, "musiccoca: head widths must be <= 256");
  MRT_REQUIRE(D <= 4096 && c.codebook >= 1 && c.codebook <= 1024 && c.rvq_depth >= 1,
              "musiccoca: d_model <= 4096, codebook_size in [1, 1024]");
  // every tensor present with its stored shape before any device work
  auto lin = [&](const std::string& n, int o, int i) {
    check_shape(w.tensor(n + ".weight"), n + ".weight", {o, i});
    check_shape(w.tensor(n + ".bias"), n + ".bias", {o});
  };
  auto ln = [&](const std::string& n) {
    check_shape(w.tensor(n + ".weight"), n + ".weight", {D});
    check_shape(w.tensor(n + ".bias"), n + ".bias", {D});
  };
  check_shape(w.tensor("token_embedding.weight"), "token_embedding.weight", {c.vocab_size, D});
  for (int i = 0; i < c.num_layers; ++i) {
    const std::string p = "text_layers." + std::to_string(i);
    ln(p + ".attn_ln");
    lin(p + ".attn.q_proj", HD, D);
    lin(p + ".attn.k_proj", HD, D);
    lin(p + ".attn.v_proj", HD, D);
    lin(p + ".attn.o_proj", D, HD);
    ln(p + ".ffn_ln");
    lin(p + ".ffn_w1", F, D);
    lin(p + ".ffn_w2", D, F);
  }
  ln("text_exit_ln");
  check_shape(w.tensor("text_pooler.query"), "text_pooler.query", {1, 1, D});
  ln("text_pooler.ln");
  lin("text_pooler.attn.q_proj", PD, D);
  lin("text_pooler.attn.k_proj", PD, D);
  lin("text_pooler.attn.v_proj", PD, D);
  lin("text_pooler.attn.o_proj", D, PD);
  check_shape(w.tensor("text_pooler.attn._per_dim_scale"), "text_pooler.attn._per_dim_scale", {c.pooler_d_head});
  const HostTensor& cb = cbs.tensor("codebooks");
  MRT_REQUIRE(cb.shape.size() == 3 && cb.shape[0] >= c.rvq_depth && cb.shape[1] == c.codebook && cb.shape[2] == D,
              "musiccoca: codebooks must be (K >= rvq_depth, codebook_size, d_model)");

  MRT_HIP_CHECK(hipSetDevice(device));
  MRT_HIP_CHECK(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking));
  MRT_HIP_CHECK(hipEventCreate(&ev_[0]));
  MRT_HIP_CHECK(hipEventCreate(&ev_[1]));
  MRT_HIP_CHECK(hipHostMalloc(reinterpret_cast<void**>(&h_stage_), 64 * 1024, hipHostMallocDefault));
  auto up = [&](const std::string& n) {
    const HostTensor& t = w.tensor(n);
    float* d = dalloc(t.numel());
    MRT_HIP_CHECK(hipMemcpy(d, t.data, t.numel() * 4, hipMemcpyHostToDevice));
    return d;
  };
  emb_table_ = up("token_embedding.weight");
  for (int i = 0; i < c.num_layers; ++i) {
    const std::string p = "text_layers." + std::to_string(i);
    ln1w_.push_back(up(p + ".attn_ln.weight"));
    ln1b_.push_back(up(p + ".attn_ln.bias"));
    qkv_.push_back(pack(w, {p + ".attn.q_proj", p + ".attn.k_proj", p + ".attn.v_proj"}, D));
    o_.push_back(pack(w, {p + ".attn.o_proj"}, HD));
    ln2w_.push_back(up(p + ".ffn_ln.weight"));
    ln2b_.push_back(up(p + ".ffn_ln.bias"));
    w1_.push_back(pack(w, {p + ".ffn_w1"}, D));
    w2_.push_back(pack(w, {p + ".ffn_w2"}, F));
  }
  exit_w_ = up("text_exit_ln.weight");
  exit_b_ = up("text_exit_ln.bias");
  pquery_ = up("text_pooler.query");
  pln_w_ = up("text_pooler.ln.weight");
  pln_b_ = up("text_pooler.ln.bias");
  pq_ = pack(w, {"text_pooler.attn.q_proj"}, D);
  pkv_ = pack(w, {"text_pooler.attn.k_proj", "text_pooler.attn.v_proj"}, D);
  po_ = pack(w, {"text_pooler.attn.o_proj"}, PD);
  {  // per-dim query scale softplus(v) / ln 2 (musiccoca.cpp:46-56, 156-160), in fp32
    const HostTensor& t = w.tensor("text_pooler.attn._per_dim_scale");
    std::vector<float> sc(c.pooler_d_head);
    for (int d = 0; d < c.pooler_d_head; ++d) {
      const float v = t.data[d];
      const float sp = std::max(v, 0.0f) + std::log1p(std::exp(-std::fabs(v)));
      sc[d] = sp / std::log(2.0f);
    }
    pscale_ = dalloc(sc.size());
    MRT_HIP_CHECK(hipMemcpy(pscale_, sc.data(), sc.size() * 4, hipMemcpyHostToDevice));
  }
  {
    const size_t n = static_cast<size_t>(c.rvq_depth) * c.codebook * D;
    codebooks_ = dalloc(n);
    MRT_HIP_CHECK(hipMemcpy(codebooks_, cb.data, n * 4, hipMemcpyHostToDevice));
  }
  ids_ = static_cast<int*>(static_cast<void*>(dalloc(L)));
  tok_ = static_cast<int*>(static_cast<void*>(dalloc(c.rvq_depth)));
  mask_ = dalloc(L);
  x_ = dalloc(static_cast<size_t>(L) * D);
  h_ = dalloc(static_cast<size_t>(L) * D);
  y_ = dalloc(static_cast<size_t>(L) * D);
  n_ = dalloc(static_cast<size_t>(L) * D);
  qkv_buf_ = dalloc(static_cast<size_t>(L) * qkv_[0].out);
  att_ = dalloc(static_cast<size_t>(L) * HD);
  f_ = dalloc(static_cast<size_t>(L) * F);
  pq_buf_ = dalloc(PD);
  pkv_buf_ = dalloc(static_cast<size_t>(L) * 2 * PD);
  patt_ = dalloc(PD);
  emb_ = dalloc(D);
  res_ = dalloc(D);
  for (int i = 0; i < c.num_layers; ++i) layer_out_.push_back(dalloc(static_cast<size_t>(L) * D));

  // the GEMM plan of one prompt (fixed: the prompt is always max_text_len rows)
  for (int i = 0; i < c.num_layers; ++i) {
    const float* xin = i == 0 ? x_ : layer_out_[i - 1];
    plan_gemm(h_, L, qkv_[i], qkv_buf_, nullptr, kActNone);
    plan_gemm(att_, L, o_[i], y_, xin, kActNone);
    plan_gemm(h_, L, w1_[i], f_, nullptr, kActGelu);
    plan_gemm(f_, L, w2_[i], layer_out_[i], y_, kActNone);
  }
  plan_gemm(pquery_, 1, pq_, pq_buf_, nullptr, kActNone);
  plan_gemm(n_, L, pkv_, pkv_buf_, nullptr, kActNone);
  plan_gemm(patt_, 1, po_, emb_, nullptr, kActNone);
  // one sub-problem per GEMM in device memory; split-K workspace
  std::vector<ConvSub> subs(steps_.size());
  size_t need = 0;
  for (size_t s = 0; s < steps_.size(); ++s) {
    ConvSub& q = subs[s];
    q = ConvSub{};  // rows (0, y, 0) -> output (y, 0), one tap at offset 0
    q.gy = steps_[s].L.hin;
    q.gx = 1;
    q.oys = q.oxs = 1;
    q.ntaps = 1;
    q.w = steps_[s].w;
    need = std::max(need, static_cast<size_t>(steps_[s].L.ksplit) * steps_[s].L.rows * steps_[s].L.cout_pad);
  }
  MRT_HIP_CHECK(hipMalloc(&subs_dev_, subs.size() * sizeof(ConvSub)));
  MRT_HIP_CHECK(hipMemcpy(subs_dev_, subs.data(), subs.size() * sizeof(ConvSub), hipMemcpyHostToDevice));
  partial_ = dalloc(std::max<size_t>(need, 1));
  for (size_t s = 0; s < steps_.size(); ++s) {
    steps_[s].L.subs = subs_dev_ + s;
    steps_[s].L.partial = partial_;
  }
}

// One GEMM y (M, out) = x (M, in) W^T + b (+ res) (act), as a one-tap
// implicit-GEMM launch (its sub-problem is uploaded with the others).
void Coca::plan_gemm(const float* x, int M, const Lin& l, float* y, const float* res, int act) {
  ConvLaunch L{};
  L.x = x;
  L.n = 1;
  L.hin = M;
  L.win = 1;
  L.cin = l.in;
  L.y = y;
  L.hout = M;
  L.wout = 1;
  L.cout = l.out;
  L.split = l.out;
  L.cout_pad = l.out_pad;
  L.bias = l.b;
  L.res = res;
  L.res_h = M;
  L.res_w = 1;
  L.rh = L.rw = 1;
  L.act_out = act;
  L.nsub = 1;
  const int tiles = (M + 63) / 64;
  L.rows = tiles * 64;
  const int blocks = tiles * (l.out_pad / 64);
  const int nk = l.in / (l.in % 32 == 0 ? 32 : 16);
  L.ksplit = blocks < 512 ? std::max(1, std::min({(512 + blocks - 1) / blocks, nk / 2, 16})) : 1;
  MRT_REQUIRE(l.in % 16 == 0, "musiccoca: GEMM inputs must be multiples of 16 wide");
  steps_.push_back(Step{L, tiles, l.out_pad / 64, l.w});
}

Coca::~Coca() {
  (void)hipSetDevice(device);
  if (stream) (void)hipStreamSynchronize(stream);
  if (graph_exec_) (void)hipGraphExecDestroy(graph_exec_);
  if (graph_) (void)hipGraphDestroy(graph_);
  if (subs_dev_) (void)hipFree(subs_dev_);
  for (void* p : allocs_) (void)hipFree(p);
  if (h_stage_) (void)hipHostFree(h_stage_);
  for (hipEvent_t e : ev_)
    if (e) (void)hipEventDestroy(e);
  if (stream) (void)hipStreamDestroy(stream);
}

// Every kernel of one prompt, from the embedding to the pooler's output
// projection (ids_ and mask_ already on the device).
void Coca::enqueue_text() {
  const CocaConfig& c = cfg;
  const int L = c.max_text_len, D = c.d_model, HD = c.num_heads * c.d_head;
  coca_embed(ids_, L, emb_table_, c.vocab_size, D, std::sqrt(static_cast<float>(D)), x_, stream);
  size_t s = 0;
  for (int i = 0; i < c.num_layers; ++i) {
    const float* xin = i == 0 ? x_ : layer_out_[i - 1];
    layer_norm_rows(xin, L, D, ln1w_[i], ln1b_[i], 1e-5f, h_, stream);
    conv_launch(steps_[s].L, steps_[s].tiles_m, steps_[s].tiles_n, stream);  // q | k | v
    ++s;
    coca_attention(qkv_buf_, 3 * HD, qkv_buf_ + HD, 3 * HD, qkv_buf_ + 2 * HD, 3 * HD, L, L, c.num_heads, c.d_head,
                   nullptr, 50.0f, mask_, att_, stream);
    conv_launch(steps_[s].L, steps_[s].tiles_m, steps_[s].tiles_n, stream);  // o + residual
    ++s;
    layer_norm_rows(y_, L, D, ln2w_[i], ln2b_[i], 1e-5f, h_, stream);
    conv_launch(steps_[s].L, steps_[s].tiles_m, steps_[s].tiles_n, stream);  // w1 + GELU
    ++s;
    conv_launch(steps_[s].L, steps_[s].tiles_m, steps_[s].tiles_n, stream);  // w2 + residual
    ++s;
  }
  // exit LayerNorm, then the pooler's own LayerNorm (musiccoca.cpp:225-231, 291-293)
  layer_norm_rows(layer_out_.back(), L, D, exit_w_, exit_b_, 1e-5f, y_, stream);
  layer_norm_rows(y_, L, D, pln_w_, pln_b_, 1e-5f, n_, stream);
  const int PD = c.num_heads * c.pooler_d_head;
  conv_launch(steps_[s].L, steps_[s].tiles_m, steps_[s].tiles_n, stream);  // pooler q (1 row)
  ++s;
  conv_launch(steps_[s].L, steps_[s].tiles_m, steps_[s].tiles_n, stream);  // pooler k | v
  ++s;
  coca_attention(pq_buf_, PD, pkv_buf_, 2 * PD, pkv_buf_ + PD, 2 * PD, 1, L, c.num_heads, c.pooler_d_head, pscale_,
                 0.0f, nullptr, patt_, stream);
  conv_launch(steps_[s].L, steps_[s].tiles_m, steps_[s].tiles_n, stream);  // pooler o
}

void Coca::embed_text(const int32_t* ids, const float* padding, float* emb) {
  const CocaConfig& c = cfg;
  const int L = c.max_text_len, D = c.d_model;
  MRT_REQUIRE(ids && padding, "musiccoca: null ids / padding");
  for (int i = 0; i < L; ++i) MRT_REQUIRE(ids[i] >= 0 && ids[i] < c.vocab_size, "musiccoca: token id out of range");
  MRT_HIP_CHECK(hipSetDevice(device));
  MRT_HIP_CHECK(hipStreamSynchronize(stream));  // staging reuse; capture starts on an idle stream
  if (calls_ == 1 && !graph_exec_) {  // second call: capture the fixed launch sequence once
    MRT_HIP_CHECK(hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal));
    try {
      enqueue_text();
    } catch (...) {
      hipGraph_t g = nullptr;
      (void)hipStreamEndCapture(stream, &g);
      if (g) (void)hipGraphDestroy(g);
      throw;
    }
    hipGraph_t g = nullptr;
    MRT_HIP_CHECK(hipStreamEndCapture(stream, &g));
    const hipError_t e = hipGraphInstantiate(&graph_exec_, g, nullptr, nullptr, 0);
    if (e != hipSuccess) {  // the next call captures again
      (void)hipGraphDestroy(g);
      graph_exec_ = nullptr;
      MRT_HIP_CHECK(e);
    }
    graph_ = g;
  }
  int32_t* hs = h_stage_;
  float* hm = reinterpret_cast<float*>(h_stage_ + L);
  std::copy(ids, ids + L, hs);
  for (int i = 0; i < L; ++i) hm[i] = padding[i] * -1e9f;  // musiccoca.cpp:279-284
  MRT_HIP_CHECK(hipMemcpyAsync(ids_, hs, L * 4, hipMemcpyHostToDevice, stream));
  MRT_HIP_CHECK(hipMemcpyAsync(mask_, hm, L * 4, hipMemcpyHostToDevice, stream));
  MRT_HIP_CHECK(hipEventRecord(ev_[0], stream));
  if (graph_exec_)
    MRT_HIP_CHECK(hipGraphLaunch(graph_exec_, stream));
  else
    enqueue_text();
  MRT_HIP_CHECK(hipEventRecord(ev_[1], stream));
  ++calls_;
  timed_ = true;
  if (emb) {
    MRT_HIP_CHECK(hipMemcpyAsync(emb, emb_, D * 4, hipMemcpyDeviceToHost, stream));
  }
  MRT_HIP_CHECK(hipStreamSynchronize(stream));
}

void Coca::tokenize(const float* emb, int32_t* tokens) {
  const CocaConfig& c = cfg;
  MRT_REQUIRE(tokens, "musiccoca: null tokens");
  MRT_HIP_CHECK(hipSetDevice(device));
  if (emb) MRT_HIP_CHECK(hipMemcpyAsync(emb_, emb, c.d_model * 4, hipMemcpyHostToDevice, stream));
  rvq_quantize(emb_, codebooks_, c.rvq_depth, c.codebook, c.d_model, res_, tok_, stream);
  MRT_HIP_CHECK(hipMemcpyAsync(h_stage_, tok_, c.rvq_depth * 4, hipMemcpyDeviceToHost, stream));
  MRT_HIP_CHECK(hipStreamSynchronize(stream));
  std::copy(h_stage_, h_stage_ + c.rvq_depth, tokens);
}

float Coca::last_ms() const {
  if (!timed_) return 0.f;
  MRT_HIP_CHECK(hipEventSynchronize(ev_[1]));
  float ms = 0.f;
  MRT_HIP_CHECK(hipEventElapsedTime(&ms, ev_[0], ev_[1]));
  return ms;
}

std::pair<const void*, size_t> Coca::buffer(int which) const {
  if (which == 0) return {emb_, static_cast<size_t>(cfg.d_model) * 4};
  if (which >= 1 && which <= cfg.num_layers)
    return {layer_out_[which - 1], static_cast<size_t>(cfg.max_text_len) * cfg.d_model * 4};
  throw Error(1, "musiccoca: unknown buffer id");
}

}  // namespace mrt
