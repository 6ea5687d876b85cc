#include "model.hpp"

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <optional>
#include <thread>

#include "batch.hpp"
#include "kernels.hpp"
#include "persist.hpp"
#include "spec.hpp"

namespace mrt {

// ---------------------------------------------------------------------------
// Relative position buckets (modules.cpp:139-174, bidirectional = false)
// ---------------------------------------------------------------------------
int relative_position_bucket(int n, int num_buckets, int max_distance) {
  if (n < 0) n = 0;
  const int eff = num_buckets;
  const int max_exact = eff / 2;
  if (n < max_exact) return n;
  const float log_ratio = std::log(static_cast<float>(max_distance) / static_cast<float>(max_exact));
  const float v = static_cast<float>(max_exact) +
                  (std::log(static_cast<float>(n) / static_cast<float>(max_exact)) / log_ratio) *
                      static_cast<float>(eff - max_exact);
  const int b = static_cast<int>(v);  // truncation, as astype(int32)
  return std::min(b, eff - 1);
}

namespace {

// Sinusoidal table in fp32 (model.cpp:54-80).
std::vector<float> sinusoid(int max_length, int features) {
  const int half = features / 2;
  MRT_REQUIRE(half > 1, "features // 2 must be >= 2 for sinusoidal PE");
  std::vector<float> data(static_cast<size_t>(max_length) * features, 0.0f);
  const float min_scale = 1.0f, max_scale = 10000.0f;
  const float scale_factor = -std::log(max_scale / min_scale) / static_cast<float>(half - 1);
  std::vector<float> div(half);
  for (int i = 0; i < half; ++i) div[i] = min_scale * std::exp(static_cast<float>(i) * scale_factor);
  for (int pos = 0; pos < max_length; ++pos) {
    float* row = &data[static_cast<size_t>(pos) * features];
    for (int i = 0; i < half; ++i) {
      const float angle = static_cast<float>(pos) * div[i];
      row[i] = std::sin(angle);
      row[half + i] = std::cos(angle);
    }
  }
  return data;
}

void expect_shape(const HostTensor& t, std::vector<int64_t> want, const std::string& key) {
  if (t.shape != want) {
    std::string got, exp;
    for (auto d : t.shape) got += std::to_string(d) + ",";
    for (auto d : want) exp += std::to_string(d) + ",";
    throw Error(1, "weight shape mismatch for " + key + ": got (" + got + ") expected (" + exp + ")");
  }
}

// Parallel fp32 -> storage conversion.
void convert(DType dt, const float* src, size_t n, void* dst) {
  if (dt == DType::F32) {
    std::memcpy(dst, src, n * 4);
    return;
  }
  uint16_t* d = static_cast<uint16_t*>(dst);
  uint16_t (*cvt)(float) = dt == DType::BF16 ? f2bf : f2h_host;
  const unsigned nt = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
  if (n < (1u << 20) || nt == 1) {
    for (size_t i = 0; i < n; ++i) d[i] = cvt(src[i]);
    return;
  }
  std::vector<std::thread> th;
  const size_t per = (n + nt - 1) / nt;
  for (unsigned t = 0; t < nt; ++t) {
    const size_t a = t * per, b = std::min(n, a + per);
    if (a >= b) break;
    th.emplace_back([=] {
      for (size_t i = a; i < b; ++i) d[i] = cvt(src[i]);
    });
  }
  for (auto& x : th) x.join();
}

}  // namespace

// Bundle keys and shapes (model.cpp:177-198, modules.cpp:342-381; Linear
// weights stored (out, in), modules.h:74-76).
std::vector<std::pair<std::string, std::vector<int64_t>>> bundle_layout(const Config& c) {
  const int64_t D = c.d_model, HD = c.hd(), F = c.d_ff, V = c.vocab_size, H = c.num_heads;
  std::vector<std::pair<std::string, std::vector<int64_t>>> out;
  out.push_back({"token_embedding.weight", {V, D}});
  out.push_back({"lm_head.weight", {V, D}});
  out.push_back({"encoder_norm.weight", {D}});
  out.push_back({"decoder_norm.weight", {D}});
  out.push_back({"temporal_rel_pos.relative_attention_bias.weight", {c.temporal_num_buckets, H}});
  out.push_back({"depth_rel_pos.relative_attention_bias.weight", {c.depth_num_buckets, H}});
  auto attn = [&](const std::string& p) {
    out.push_back({p + ".q_proj.weight", {HD, D}});
    out.push_back({p + ".k_proj.weight", {HD, D}});
    out.push_back({p + ".v_proj.weight", {HD, D}});
    out.push_back({p + ".o_proj.weight", {D, HD}});
  };
  auto ffn = [&](const std::string& p) {
    out.push_back({p + ".wi_0.weight", {F, D}});
    out.push_back({p + ".wi_1.weight", {F, D}});
    out.push_back({p + ".wo.weight", {D, F}});
  };
  for (int i = 0; i < c.num_encoder_layers; ++i) {
    const std::string p = "encoder_layers." + std::to_string(i);
    out.push_back({p + ".pre_attn_norm.weight", {D}});
    attn(p + ".self_attn");
    out.push_back({p + ".pre_ffn_norm.weight", {D}});
    ffn(p + ".ffn");
  }
  for (int i = 0; i < c.num_temporal_layers; ++i) {
    const std::string p = "temporal_layers." + std::to_string(i);
    out.push_back({p + ".pre_self_attn_norm.weight", {D}});
    attn(p + ".self_attn");
    out.push_back({p + ".pre_cross_attn_norm.weight", {D}});
    attn(p + ".cross_attn");
    out.push_back({p + ".pre_ffn_norm.weight", {D}});
    ffn(p + ".ffn");
  }
  for (int i = 0; i < c.num_depth_layers; ++i) {
    const std::string p = "depth_layers." + std::to_string(i);
    out.push_back({p + ".pre_self_attn_norm.weight", {D}});
    attn(p + ".self_attn");
    out.push_back({p + ".pre_ffn_norm.weight", {D}});
    ffn(p + ".ffn");
  }
  return out;
}

// ---------------------------------------------------------------------------
// Model
// ---------------------------------------------------------------------------

const void* Model::upload(const std::vector<float>& host) {
  const size_t bytes = host.size() * esz;
  void* d = nullptr;
  MRT_HIP_CHECK(hipMalloc(&d, std::max<size_t>(bytes, 256)));
  allocs_.push_back(d);
  std::vector<uint8_t> tmp(bytes);
  convert(dt, host.data(), host.size(), tmp.data());
  MRT_HIP_CHECK(hipMemcpy(d, tmp.data(), bytes, hipMemcpyHostToDevice));
  weight_bytes += bytes;
  return d;
}

const void* Model::upload_i32(const std::vector<int>& host) {
  void* d = nullptr;
  MRT_HIP_CHECK(hipMalloc(&d, host.size() * 4));
  allocs_.push_back(d);
  MRT_HIP_CHECK(hipMemcpy(d, host.data(), host.size() * 4, hipMemcpyHostToDevice));
  return d;
}

Model::Model(const TensorSource& src, const Config& c, DType dtype, int dev)
    : cfg(c), dt(dtype), device(dev), esz(dtype_size(dtype)) {
  MRT_REQUIRE(cfg.d_kv == 64, "this backend requires d_kv == 64");
  MRT_REQUIRE(cfg.d_model % 64 == 0 && cfg.d_ff % 64 == 0, "d_model and d_ff must be multiples of 64");
  MRT_REQUIRE(cfg.num_heads >= 1 && cfg.vocab_size >= 2, "bad config");
  MRT_REQUIRE(cfg.max_encoder_length >= 1 && cfg.rvq_depth >= 1, "bad config");
  const int64_t D = cfg.d_model, HD = cfg.hd(), F = cfg.d_ff, V = cfg.vocab_size, H = cfg.num_heads;
  // Every key and shape is checked before the device is touched.
  for (const auto& ks : bundle_layout(cfg)) expect_shape(src.tensor(ks.first), ks.second, ks.first);
  MRT_HIP_CHECK(hipSetDevice(device));

  auto get = [&](const std::string& key, std::vector<int64_t> shape) -> const HostTensor& {
    const HostTensor& t = src.tensor(key);
    expect_shape(t, shape, key);
    return t;
  };
  auto vec = [&](const std::string& key, std::vector<int64_t> shape) {
    const HostTensor& t = get(key, shape);
    return std::vector<float>(t.data, t.data + t.numel());
  };
  // Row-concatenate several (rows_i, D) matrices.
  auto cat = [&](const std::vector<std::pair<std::string, int64_t>>& parts, int64_t cols) {
    size_t total = 0;
    for (auto& p : parts) total += static_cast<size_t>(p.second * cols);
    std::vector<float> out;
    out.reserve(total);
    for (auto& p : parts) {
      const HostTensor& t = get(p.first, {p.second, cols});
      out.insert(out.end(), t.data, t.data + t.numel());
    }
    return out;
  };
  // wi_0 / wi_1 packed in 32-row groups [gate 32 | up 32].
  auto pack_geglu = [&](const std::string& prefix) {
    const HostTensor& w0 = get(prefix + ".wi_0.weight", {F, D});
    const HostTensor& w1 = get(prefix + ".wi_1.weight", {F, D});
    std::vector<float> out(static_cast<size_t>(2 * F * D));
    for (int64_t g = 0; g < F / 32; ++g) {
      std::memcpy(&out[(size_t)(g * 64) * D], w0.data + (size_t)(g * 32) * D, sizeof(float) * 32 * D);
      std::memcpy(&out[(size_t)(g * 64 + 32) * D], w1.data + (size_t)(g * 32) * D, sizeof(float) * 32 * D);
    }
    return out;
  };

  emb = upload(vec("token_embedding.weight", {V, D}));
  lm_head = upload(vec("lm_head.weight", {V, D}));
  {
    // The fp32 table is cast to the model dtype before the add (model.cpp:232-236);
    // the fp32 values stay on the host for position_embedding.
    pe_host_ = sinusoid(cfg.max_encoder_length, cfg.d_model);
    pe = upload(pe_host_);
  }
  enc_norm = upload(vec("encoder_norm.weight", {D}));
  dec_norm = upload(vec("decoder_norm.weight", {D}));
  tbias = upload(vec("temporal_rel_pos.relative_attention_bias.weight", {cfg.temporal_num_buckets, H}));
  dbias = upload(vec("depth_rel_pos.relative_attention_bias.weight", {cfg.depth_num_buckets, H}));
  {
    std::vector<int> tb(kBucketTable), db(kBucketTable);
    for (int n = 0; n < kBucketTable; ++n) {
      tb[n] = relative_position_bucket(n, cfg.temporal_num_buckets, cfg.temporal_max_distance);
      db[n] = relative_position_bucket(n, cfg.depth_num_buckets, cfg.depth_max_distance);
    }
    tbuckets = static_cast<const int*>(upload_i32(tb));
    dbuckets = static_cast<const int*>(upload_i32(db));
    // the persistent kernels read row pos < kMaxPersistLen of these tables
    static_assert(kBiasRows >= kMaxPersistLen, "bias rows must cover every persistent ring position");
    const size_t n_rows = static_cast<size_t>(H) * kBiasRows * (kBiasRows + 1) / 2;
    void* t = nullptr;
    void* d = nullptr;
    MRT_HIP_CHECK(hipMalloc(&t, n_rows * esz));
    allocs_.push_back(t);
    MRT_HIP_CHECK(hipMalloc(&d, n_rows * esz));
    allocs_.push_back(d);
    precompute_biases(0, kBiasRows, t);
    precompute_biases(1, kBiasRows, d);
    tbias_rows = t;
    dbias_rows = d;
  }

  for (int i = 0; i < cfg.num_encoder_layers; ++i) {
    const std::string p = "encoder_layers." + std::to_string(i);
    EncoderLayerW w{};
    w.norm_attn = upload(vec(p + ".pre_attn_norm.weight", {D}));
    w.wqkv = upload(cat({{p + ".self_attn.q_proj.weight", HD},
                         {p + ".self_attn.k_proj.weight", HD},
                         {p + ".self_attn.v_proj.weight", HD}}, D));
    w.wo = upload(vec(p + ".self_attn.o_proj.weight", {D, HD}));
    w.norm_ff = upload(vec(p + ".pre_ffn_norm.weight", {D}));
    w.w01 = upload(pack_geglu(p + ".ffn"));
    w.wo2 = upload(vec(p + ".ffn.wo.weight", {D, F}));
    enc.push_back(w);
  }
  // Decoder stacks are stored per weight kind with layers back to back, so a
  // layer's weights sit at base + layer * (one layer's elements).
  std::vector<std::pair<std::string, int64_t>> cross_parts;
  auto decoder_stack = [&](const std::string& prefix, int n, bool temporal, std::vector<DecoderLayerW>& out) {
    std::vector<std::vector<float>> norm_sa, wqkv, wo, norm_ca, wq_c, wo_c, norm_ff, w01, wo2;
    for (int i = 0; i < n; ++i) {
      const std::string p = prefix + "." + std::to_string(i);
      norm_sa.push_back(vec(p + ".pre_self_attn_norm.weight", {D}));
      wqkv.push_back(cat({{p + ".self_attn.q_proj.weight", HD},
                          {p + ".self_attn.k_proj.weight", HD},
                          {p + ".self_attn.v_proj.weight", HD}}, D));
      wo.push_back(vec(p + ".self_attn.o_proj.weight", {D, HD}));
      if (temporal) {
        norm_ca.push_back(vec(p + ".pre_cross_attn_norm.weight", {D}));
        wq_c.push_back(vec(p + ".cross_attn.q_proj.weight", {HD, D}));
        wo_c.push_back(vec(p + ".cross_attn.o_proj.weight", {D, HD}));
        cross_parts.push_back({p + ".cross_attn.k_proj.weight", HD});
        cross_parts.push_back({p + ".cross_attn.v_proj.weight", HD});
      }
      norm_ff.push_back(vec(p + ".pre_ffn_norm.weight", {D}));
      w01.push_back(pack_geglu(p + ".ffn"));
      wo2.push_back(vec(p + ".ffn.wo.weight", {D, F}));
    }
    out.assign(n, DecoderLayerW{});
    auto place = [&](std::vector<std::vector<float>>& parts, const void* DecoderLayerW::*field) {
      if (parts.empty()) return;
      const size_t per = parts[0].size();
      std::vector<float> all;
      all.reserve(per * parts.size());
      for (auto& v : parts) {
        all.insert(all.end(), v.begin(), v.end());
        std::vector<float>().swap(v);
      }
      const char* base = static_cast<const char*>(upload(all));
      for (int i = 0; i < n; ++i) out[i].*field = base + static_cast<size_t>(i) * per * esz;
    };
    place(norm_sa, &DecoderLayerW::norm_sa);
    place(wqkv, &DecoderLayerW::wqkv);
    place(wo, &DecoderLayerW::wo);
    place(norm_ca, &DecoderLayerW::norm_ca);
    place(wq_c, &DecoderLayerW::wq_c);
    place(wo_c, &DecoderLayerW::wo_c);
    place(norm_ff, &DecoderLayerW::norm_ff);
    place(w01, &DecoderLayerW::w01);
    place(wo2, &DecoderLayerW::wo2);
  };
  decoder_stack("temporal_layers", cfg.num_temporal_layers, true, tmp);
  if (!cross_parts.empty()) wkv_cross = upload(cat(cross_parts, D));
  decoder_stack("depth_layers", cfg.num_depth_layers, false, dep);
}

Model::~Model() {
  (void)hipSetDevice(device);
  for (void* p : allocs_) (void)hipFree(p);
  if (embed_ids_host_) (void)hipHostFree(embed_ids_host_);
}

void Model::embed_tokens(const int32_t* ids, int n, void* out, hipStream_t s) {
  MRT_REQUIRE(n >= 0, "token_embedding: negative id count");
  for (int i = 0; i < n; ++i)
    MRT_REQUIRE(ids[i] >= 0 && ids[i] < cfg.vocab_size, "token_embedding: token id out of range");
  if (n == 0) return;
  MRT_HIP_CHECK(hipSetDevice(device));
  std::lock_guard<std::mutex> lock(embed_mu_);
  if (embed_ids_dev_ == nullptr) {
    void* d = nullptr;
    MRT_HIP_CHECK(hipMalloc(&d, kEmbedChunk * sizeof(int)));
    allocs_.push_back(d);
    embed_ids_dev_ = static_cast<int*>(d);
    MRT_HIP_CHECK(hipHostMalloc(reinterpret_cast<void**>(&embed_ids_host_), kEmbedChunk * sizeof(int),
                                hipHostMallocDefault));
  }
  const size_t row = static_cast<size_t>(cfg.d_model) * esz;
  for (int i0 = 0; i0 < n; i0 += kEmbedChunk) {
    const int k = std::min(kEmbedChunk, n - i0);
    std::memcpy(embed_ids_host_, ids + i0, static_cast<size_t>(k) * sizeof(int));
    MRT_HIP_CHECK(hipMemcpyAsync(embed_ids_dev_, embed_ids_host_, static_cast<size_t>(k) * sizeof(int),
                                 hipMemcpyHostToDevice, s));
    embed_rows(dt, emb, cfg.d_model, embed_ids_dev_, k, static_cast<char*>(out) + i0 * row, s);
    MRT_HIP_CHECK(hipStreamSynchronize(s));  // the staging is reused by the next chunk and call
  }
}

void Model::position_embedding(int seq_len, float* out) const {
  MRT_REQUIRE(seq_len >= 0, "position_embedding: negative seq_len");
  if (seq_len > cfg.max_encoder_length) throw Error(1, "seq_len exceeds max_encoder_length");
  if (seq_len == 0) return;
  MRT_HIP_CHECK(hipSetDevice(device));
  MRT_HIP_CHECK(hipMemcpy(out, pe_host_.data(), static_cast<size_t>(seq_len) * cfg.d_model * sizeof(float),
                          hipMemcpyHostToDevice));
}

// ---------------------------------------------------------------------------
// State
// ---------------------------------------------------------------------------

void* State::dalloc(size_t bytes) {
  void* d = nullptr;
  MRT_HIP_CHECK(hipMalloc(&d, std::max<size_t>(bytes, 256)));
  allocs_.push_back(d);
  return d;
}

State::State(Model& model, int rows_, int max_frames, int enc_len)
    : m(model), rows(rows_), F(max_frames), S(enc_len) {
  const Config& c = m.cfg;
  MRT_REQUIRE(rows == 2, "rows must be 2 (one CFG stream)");
  MRT_REQUIRE(F >= 1 && F < Model::kBucketTable, "max_frames out of range");
  MRT_REQUIRE(S >= 1 && S <= c.max_encoder_length, "enc_len must be in [1, max_encoder_length]");
  MRT_HIP_CHECK(hipSetDevice(m.device));
  MRT_HIP_CHECK(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking));
  const size_t D = c.d_model, HD = c.hd(), FF = c.d_ff, H = c.num_heads, L = c.rvq_depth;
  const size_t M = static_cast<size_t>(rows) * S, e = esz();
  d_enc_tok = static_cast<int*>(dalloc(M * 4));
  ex = dalloc(M * D * e);
  exn = dalloc(M * D * e);
  eqkv = dalloc(M * 3 * HD * e);
  eattn = dalloc(M * HD * e);
  effh = dalloc(M * FF * e);
  enc_out = dalloc(M * D * e);
  cross = dalloc(static_cast<size_t>(c.num_temporal_layers) * 2 * rows * H * S * 64 * e);
  tkv = dalloc(static_cast<size_t>(c.num_temporal_layers) * 2 * rows * H * F * 64 * e);
  dkv = dalloc(static_cast<size_t>(c.num_depth_layers) * 2 * rows * H * L * 64 * e);
  x = dalloc(rows * D * e);
  q = dalloc(rows * HD * e);
  attn = dalloc(rows * HD * e);
  ffh = dalloc(rows * FF * e);
  t_in = dalloc(rows * D * e);
  t_out = dalloc(rows * D * e);
  d_in = dalloc(rows * D * e);
  fsum = dalloc(rows * D * e);
  max_slice = c.vocab_size;
  slice = static_cast<float*>(dalloc(static_cast<size_t>(rows) * c.vocab_size * 4));
  nsplit = cross_attn_splits(S);
  part = static_cast<float*>(dalloc(static_cast<size_t>(rows) * H * nsplit * 66 * 4));
  d_tokens = static_cast<int*>(dalloc(static_cast<size_t>(F) * L * 4));
  d_teacher = static_cast<int*>(dalloc(static_cast<size_t>(F) * L * 4));
  d_seed = static_cast<uint64_t*>(dalloc(8));
  h_pinned_n = std::max<size_t>(M, static_cast<size_t>(F) * L + F) + 2;  // tokens + per-frame accepted counts
  MRT_HIP_CHECK(hipHostMalloc(reinterpret_cast<void**>(&h_pinned), h_pinned_n * 4, hipHostMallocDefault));
  MRT_HIP_CHECK(hipHostMalloc(reinterpret_cast<void**>(&h_err_), 64, hipHostMallocDefault));
  *h_err_ = 0;
  MRT_HIP_CHECK(hipHostMalloc(reinterpret_cast<void**>(&h_seed_), 64, hipHostMallocDefault));
  d_prof_ = static_cast<uint64_t*>(dalloc(static_cast<size_t>(F) * 4 * sizeof(uint64_t)));
  MRT_HIP_CHECK(hipHostMalloc(reinterpret_cast<void**>(&h_prof_), static_cast<size_t>(F) * 4 * sizeof(uint64_t),
                              hipHostMallocDefault));
  {  // rows of the full-sequence depth pass and the speculative verification pass (2 L rows)
    const size_t R2 = 2 * L;
    sx_ = dalloc(R2 * D * e);
    sxn_ = dalloc(R2 * std::max(D, FF) * e);
    sqkv_ = dalloc(R2 * 3 * HD * e);
    satt_ = dalloc(R2 * HD * e);
    sffh_ = dalloc(R2 * FF * e);
  }
  if (m.dt == DType::BF16) {  // speculative decoding
    const size_t R2 = 2 * L;
    d_drafts_ = static_cast<int*>(dalloc(static_cast<size_t>(F) * L * 4));
    sq_ = dalloc(R2 * HD * e);
    slog_ = static_cast<float*>(dalloc(R2 * 1024 * 4));
    sdrawn_ = static_cast<int*>(dalloc(L * 4));
    sdecided_ = static_cast<int*>(dalloc(static_cast<size_t>(F) * 4));
    sfm_ = dalloc(rows * D * e);
  }
  const char* path = std::getenv("MRT_DECODE_PATH");
  if (!(path && std::string(path) == "layers")) setup_persistent();
}

// The persistent path needs: head dim 64 (checked by Model), every GEMV input
// <= 1024 wide except d_ff <= 3072, GEMV inputs in whole 16-byte chunks
// (d_model % 8 == 0), rings of <= 64 slots, and a grid of
// H * bph workgroups (bph >= 8) that fits on the device.
void State::setup_persistent() {
  const Config& c = m.cfg;
  int num_cu = 0;
  MRT_HIP_CHECK(hipDeviceGetAttribute(&num_cu, hipDeviceAttributeMultiprocessorCount, m.device));
  int bph = 0;
  const int grid = persist_grid(c.num_heads, num_cu, &bph);
  // Every workgroup must own rows of the d_model and d_ff phases (the launch
  // epoch advances once data from all workgroups has been seen).
  const bool ok = grid > 0 && c.d_model <= 1024 && c.d_model % 8 == 0 && c.hd() <= 1024 && c.d_ff <= kMaxPersistK &&
                  c.d_ff % 32 == 0 &&
                  F <= kMaxPersistLen && c.rvq_depth <= kMaxPersistLen && S <= kMaxCrossChunk * bph && c.d_model >= grid &&
                  c.d_ff >= grid;
  if (!ok) return;
  lds_t_ = persist_prepare(m.dt, PersistKernel::Temporal, m.device);
  lds_d_ = persist_prepare(m.dt, PersistKernel::Depth, m.device);
  if (lds_t_ == 0 || lds_d_ == 0) return;
  persist_grid_ = grid;
  bph_ = bph;
  // The frame kernel keeps the depth history in LDS and numbers the phases of
  // a whole frame in one tag space.
  const int codes = 16 * (c.num_temporal_layers + 1) + 16 * c.rvq_depth * (c.num_depth_layers + 1);
  const char* fk = std::getenv("MRT_FRAME_KERNEL");
  if (!(fk && std::string(fk) == "0") && c.num_depth_layers * c.rvq_depth <= kMaxResidentSlots &&
      codes <= (1 << kTagShift)) {
    lds_f_ = persist_prepare(m.dt, PersistKernel::Frame, m.device);
    frame_kernel_ = lds_f_ > 0;
    // the levels after a speculative verification pass run in one launch too
    if (frame_kernel_) lds_l_ = persist_prepare(m.dt, PersistKernel::Levels, m.device);
  }
  const size_t H = c.num_heads;
  // Tagged hand-off words: x, q, k, v, at, h vectors, cross partials, logits,
  // then the epoch counter and the error flag.
  const size_t vec = kLLVecWords;
  const size_t part = static_cast<size_t>(H) * kMaxBph * 2 * 66;
  const size_t logit = 2 * static_cast<size_t>(c.vocab_size);
  ll_words_ = 6 * vec + part + logit + 64;
  ll_block_ = dalloc(ll_words_ * sizeof(uint64_t));
  noise_ = static_cast<float*>(dalloc(static_cast<size_t>(F) * c.rvq_depth * 1024 * sizeof(float)));
  reset_handoff();
  auto stack = [&](const std::vector<DecoderLayerW>& ws, bool temporal) {
    DecStack d{};
    if (ws.empty()) return d;
    const DecoderLayerW& w = ws[0];
    d.norm_sa = w.norm_sa;
    d.wqkv = w.wqkv;
    d.wo = w.wo;
    d.norm_ca = w.norm_ca;
    d.wq_c = w.wq_c;
    d.wo_c = w.wo_c;
    d.norm_ff = w.norm_ff;
    d.w01 = w.w01;
    d.wo2 = w.wo2;
    d.cross = temporal ? ck(0) : nullptr;
    d.ring = temporal ? tk(0) : dk(0);
    return d;
  };
  tstack_ = stack(m.tmp, true);
  dstack_ = stack(m.dep, false);
  // First-poll delays per PollSite and stack (temporal, depth), measured on
  // MI355X at the benchmark dims (bf16 frame kernel, greedy per-site sweeps
  // over 0..32, each value timed next to the current best in one process):
  // the layer inputs of the q/k/v, output and gated-GELU projections and the
  // head logits are polled at once, the gated-GELU output after 24 rounds (its
  // producers finish last), the cross-attention query input after 16, the
  // cross partials' query and the head input after 8, the rest after 4.  A
  // separate sweep per stack found the same values for both.  MRT_POLL_DELAY=n
  // sets every site, MRT_POLL_DELAYS a comma-separated list in PollSite order
  // for both stacks, MRT_POLL_DELAYS_T / MRT_POLL_DELAYS_D for one stack
  // (missing entries keep their value).
  static constexpr uint8_t kDefaultDelay[kPollSites] = {0, 4, 0, 16, 8, 4, 4, 0, 24, 8, 0, 4};
  auto parse = [](const char* d, uint8_t* dl) {
    const char* c = d;
    for (int i = 0; i < kPollSites; ++i) {
      char* end = nullptr;
      const long v = std::strtol(c, &end, 10);
      if (end != c) dl[i] = static_cast<uint8_t>(std::max(0L, std::min(255L, v)));
      if (*end != ',') break;
      c = end + 1;
    }
  };
  for (int k = 0; k < 2; ++k) {
    uint8_t* dl = poll_delay_[k];
    std::copy(kDefaultDelay, kDefaultDelay + kPollSites, dl);
    if (const char* d = std::getenv("MRT_POLL_DELAY"))
      std::fill(dl, dl + kPollSites, static_cast<uint8_t>(std::max(0, std::min(255, std::atoi(d)))));
    if (const char* d = std::getenv("MRT_POLL_DELAYS")) parse(d, dl);
    if (const char* d = std::getenv(k == 0 ? "MRT_POLL_DELAYS_T" : "MRT_POLL_DELAYS_D")) parse(d, dl);
  }
  if (const char* q = std::getenv("MRT_QKV_TABLE")) qkv_table_on_ = std::string(q) != "0";
  if (const char* pr = std::getenv("MRT_PROFILE_DECODE")) profile_ = pr[0] != '\0';
  if (std::getenv("MRT_TRACE_PHASES")) {
    d_trace_ = static_cast<uint64_t*>(dalloc(2 * kTraceSlots * sizeof(uint64_t)));
    MRT_HIP_CHECK(hipMemset(d_trace_, 0, 2 * kTraceSlots * sizeof(uint64_t)));
  }
}

// Per-phase timeline of one temporal and one depth step (frame 1, level 1).
void State::print_trace() {
  if (!d_trace_) return;
  std::vector<uint64_t> t(2 * kTraceSlots);
  MRT_HIP_CHECK(hipMemcpy(t.data(), d_trace_, t.size() * sizeof(uint64_t), hipMemcpyDeviceToHost));
  const char* names[2] = {"temporal_step", "depth_step"};
  for (int w = 0; w < 2; ++w) {
    const uint64_t* r = t.data() + w * kTraceSlots;
    const uint64_t t0 = r[kTraceStart];
    if (!t0) continue;
    // Raw timeline: deltas between consecutive trace points (first 48).
    std::string line;
    uint64_t prev = t0;
    int nb = 0;
    for (int k = 0; k < 400 && r[k]; ++k, ++nb) {
      if (k < (w == 0 ? 48 : 100)) {
        char buf[32];
        std::snprintf(buf, sizeof buf, " %.2f", (r[k] - prev) * 0.01);
        line += buf;
      }
      prev = r[k];
    }
    std::fprintf(stderr, "[mrt] %s: %d points, total %.2f us (to final arrival %.2f us); deltas us:%s\n", names[w], nb,
                 (r[kTraceDone] - t0) * 0.01, (r[kTraceEnd] - t0) * 0.01, line.c_str());
    // per-wave poll completion of the first loads, relative to the load's start
    std::string pw;
    for (int k = 0; k < 16 && r[400 + k]; ++k) {
      pw += " [";
      for (int wv = 0; wv < 4; ++wv) {
        const uint64_t v = r[420 + 4 * k + wv];
        char buf[32];
        std::snprintf(buf, sizeof buf, "%s%.2f", wv ? " " : "", v ? (double)(int64_t)(v - r[400 + k]) * 0.01 : -1.0);
        pw += buf;
      }
      pw += "]";
    }
    std::fprintf(stderr, "[mrt] %s: per-wave poll done (us after load start):%s\n", names[w], pw.c_str());
    if (r[490]) {  // inside the draw: v, argmax, count, [fallback], publish, then radix passes 1-4
      std::string dl;
      uint64_t pv = r[kTraceEnd];
      for (int k = 490; k < 499 && r[k]; ++k) {
        if (k == 495) pv = r[492];  // radix passes start after the count
        char buf[32];
        std::snprintf(buf, sizeof buf, " %.2f", (r[k] - pv) * 0.01);
        dl += buf;
        pv = r[k];
      }
      std::fprintf(stderr, "[mrt] %s: draw deltas us (from gather end):%s\n", names[w], dl.c_str());
    }
  }
}

LLBufs State::ll_bufs(int stack) const {
  uint64_t* b = static_cast<uint64_t*>(ll_block_);
  const size_t vec = kLLVecWords;
  LLBufs l;
  l.x = b;
  l.q = b + vec;
  l.k = b + 2 * vec;
  l.v = b + 3 * vec;
  l.at = b + 4 * vec;
  l.h = b + 5 * vec;
  l.part = b + 6 * vec;
  l.logit = l.part + static_cast<size_t>(m.cfg.num_heads) * kMaxBph * 2 * 66;
  uint64_t* tail = l.logit + 2 * static_cast<size_t>(m.cfg.vocab_size);
  l.seq = reinterpret_cast<uint32_t*>(tail);
  l.tok = tail + 16;
  l.err = reinterpret_cast<int*>(tail + 32);
  std::memcpy(l.delay, poll_delay_[stack], kPollSites);
  return l;
}

// Zero every hand-off word and start the epoch at 1, so no zeroed word can
// carry a live tag.
void State::reset_handoff() {
  MRT_HIP_CHECK(hipMemsetAsync(ll_block_, 0, ll_words_ * sizeof(uint64_t), stream));
  const uint32_t one = 1;
  MRT_HIP_CHECK(hipMemcpyAsync(ll_bufs().seq, &one, sizeof(one), hipMemcpyHostToDevice, stream));
  MRT_HIP_CHECK(hipStreamSynchronize(stream));
  epochs_used_ = 0;
}

// Each persistent launch advances the epoch by one; tags keep its low 20
// bits.  Before those wrap, every hand-off word is zeroed and the epoch
// restarts (outside any capture: callers reserve before enqueueing).
void State::reserve_epochs(uint32_t n) {
  if (epochs_used_ + n + 2 >= kEpochPeriod) reset_handoff();
  epochs_used_ += n;
}

int State::spec_count(const GenOpts& o) const {
  if (!spec_drafts_) return 0;
  return o.spec_frames > 0 ? std::min(o.spec_frames, o.num_frames) : o.num_frames;
}

int State::decode_launches(const GenOpts& o) const {
  // speculative frames: the temporal step, then one launch of the open levels
  // (or, without that kernel, L - 1 depth steps)
  const int ns = spec_count(o);
  return ns * (lds_l_ > 0 ? 2 : o.rvq_depth) + (o.num_frames - ns) * (frame_kernel_ ? 1 : 1 + o.rvq_depth);
}

StepArgs State::temporal_args(const void* in, int f, void* out) const {
  const Config& c = m.cfg;
  StepArgs a{};
  if (d_trace_ && f == 1) a.trace = d_trace_;
  a.st = tstack_;
  a.nlayers = c.num_temporal_layers;
  a.cross = 1;
  a.D = c.d_model;
  a.HD = c.hd();
  a.H = c.num_heads;
  a.F = c.d_ff;
  a.bph = bph_;
  a.pos = f;
  a.Lmax = F;
  a.bias_rows = m.tbias_rows;
  a.in = in;
  a.out = out;
  a.S = S;
  a.ll = ll_bufs(0);
  return a;
}

StepArgs State::depth_args(const void* in, int l, const void* head_w, int head_rows, float* logits,
                           float* rec_slice) const {
  const Config& c = m.cfg;
  StepArgs a{};
  a.st = dstack_;
  a.nlayers = c.num_depth_layers;
  a.cross = 0;
  a.D = c.d_model;
  a.HD = c.hd();
  a.H = c.num_heads;
  a.F = c.d_ff;
  a.bph = bph_;
  a.pos = l;
  a.Lmax = c.rvq_depth;
  a.bias_rows = m.dbias_rows;
  a.in = in;
  a.S = S;
  a.dec_norm = m.dec_norm;
  a.head_w = head_w;
  a.head_rows = head_rows;
  a.logits = logits;
  a.rec_slice = rec_slice;
  a.ll = ll_bufs(1);
  return a;
}

void State::launch_temporal_p(const void* in, int f, void* out, const void* bias) {
  StepArgs a = temporal_args(in, f, out);
  a.bias_row = bias;
  if (d_trace_ && f == 1) a.trace = d_trace_;
  launch_step(m.dt, a, persist_grid_, lds_t_, stream);
}

void State::launch_depth_p(const void* in, int l, const void* head_w, int head_rows, float* logits,
                           float* rec_slice, const void* bias) {
  StepArgs a = depth_args(in, l, head_w, head_rows, logits, rec_slice);
  a.bias_row = bias;
  launch_step(m.dt, a, persist_grid_, lds_d_, stream);
}

// Frame f of the decode loop as one launch: temporal step on t_in, 16 depth
// steps with on-device draws; the frame mean lands in t_in.
void State::launch_frame_p(const GenOpts& o, int f) {
  const Config& c = m.cfg;
  const int D = c.d_model, C = o.codebook, L = o.rvq_depth;
  const size_t row_bytes = static_cast<size_t>(rows) * D * esz();
  FrameArgs fa{};
  fa.t = temporal_args(t_in, f, nullptr);
  if (d_trace_ && f == 1) fa.t.trace = d_trace_;
  const void* head = static_cast<const char*>(m.lm_head) + static_cast<size_t>(o.codec_offset) * D * esz();
  fa.d = depth_args(nullptr, 0, head, C, nullptr, nullptr);
  if (d_trace_ && f == 1) fa.d.trace = d_trace_ + kTraceSlots;
  fa.d.sp = SampleParams{o.guidance_weight, o.temperature, o.top_k, C, o.codec_offset, L, d_seed};
  fa.d.frame = f;
  fa.d.teacher = o.teacher ? d_teacher : nullptr;
  fa.d.tokens = d_tokens;
  fa.d.drawn = o.record_drawn;
  fa.d.emb = m.emb;
  fa.d.fmean = t_in;
  fa.d.noise = noise_ + static_cast<size_t>(f) * L * C;
  fa.codebook = C;
  fa.levels = L;
  fa.rec_slices = o.record_slices ? o.record_slices + static_cast<size_t>(f) * L * rows * C : nullptr;
  fa.rec_temporal = o.record_temporal ? static_cast<char*>(o.record_temporal) + f * row_bytes : nullptr;
  fa.qkv_table = qkv_table_;
  fa.prof = profile_ ? d_prof_ : nullptr;
  launch_frame(m.dt, fa, persist_grid_, lds_f_, stream);
}

// Decode loop on the persistent kernels (decode.cpp:339-486).  Frame 0 feeds
// emb(PAD = 0) on both rows; the Gumbel noise of every draw is tabulated
// first.  Without the frame kernel each step is one launch and each draw
// runs in the sampling kernel.
void State::enqueue_decode_p(const GenOpts& o) {
  const Config& c = m.cfg;
  const int D = c.d_model, C = o.codebook, L = o.rvq_depth;
  embed_fill(m.dt, m.emb, D, 0, rows, t_in, stream);
  gumbel_table(d_seed, o.num_frames, L, C, noise_, stream);
  SampleParams sp{o.guidance_weight, o.temperature, o.top_k, C, o.codec_offset, L, d_seed};
  for (int f = 0; f < o.num_frames; ++f) enqueue_plain_frame(o, f, sp);
}

// Frame f of the plain persistent decode: one frame-kernel launch, or one
// launch per step plus the sampling kernel; t_in holds the frame's input
// (emb(PAD) or the previous frame mean) and receives this frame's mean.
void State::enqueue_plain_frame(const GenOpts& o, int f, const SampleParams& sp) {
  const Config& c = m.cfg;
  const int D = c.d_model, C = o.codebook, L = o.rvq_depth;
  const size_t row_bytes = static_cast<size_t>(rows) * D * esz();
  if (frame_kernel_) {
    launch_frame_p(o, f);
  } else {
    launch_temporal_p(t_in, f, t_out);
    if (o.record_temporal) copy(static_cast<char*>(o.record_temporal) + f * row_bytes, t_out, row_bytes);
    for (int l = 0; l < L; ++l) {
      const char* head = static_cast<const char*>(m.lm_head) + static_cast<size_t>(o.codec_offset + C * l) * D * esz();
      float* rec = o.record_slices ? o.record_slices + (static_cast<size_t>(f) * L + l) * rows * C : nullptr;
      launch_depth_p(l == 0 ? t_out : d_in, l, head, C, slice, rec);
      sample_level(m.dt, slice, sp, f, l, f * L + l, o.teacher ? d_teacher : nullptr, d_tokens, o.record_drawn,
                   m.emb, D, d_in, fsum, t_in, stream);
    }
  }
  if (o.record_frame_mean) copy(static_cast<char*>(o.record_frame_mean) + f * row_bytes, t_in, row_bytes);
}

// Speculation runs when asked for, on the bf16 persistent path, with drafts
// from a previous call of the same frame count and no teacher or per-draw
// records (the reference also speculates only once a chunk exists,
// system.cpp:244-256).
bool State::speculating(const GenOpts& o) const {
  return o.speculative && m.dt == DType::BF16 && persistent() && o.teacher == nullptr && o.record_drawn == nullptr &&
         o.record_frame_mean == nullptr && 2 * o.rvq_depth <= kBatchRows && o.rvq_depth == m.cfg.rvq_depth;
}

// The decode loop with speculative depth decoding (decode.cpp:380-446).  Per
// frame: the temporal step; one causal pass over [temporal_out, emb(draft
// 0..L-2)] (depth_forward_full, model.cpp:243-268) writing the depth K/V of
// every position and every level's logits; every level drawn with its own
// noise; the drafts accepted up to the first disagreement (whose draw is the
// token); then the remaining levels as depth steps with draws (each skips
// itself when its level is already decided); the frame mean of the L tokens.
void State::enqueue_decode_spec(const GenOpts& o) {
  const Config& c = m.cfg;
  const DType dt = m.dt;
  const int D = c.d_model, HD = c.hd(), FF = c.d_ff, H = c.num_heads, C = o.codebook, L = o.rvq_depth;
  const int R2 = 2 * L;
  const size_t row_bytes = static_cast<size_t>(rows) * D * esz();
  embed_fill(dt, m.emb, D, 0, rows, t_in, stream);
  gumbel_table(d_seed, o.num_frames, L, C, noise_, stream);
  SampleParams sp{o.guidance_weight, o.temperature, o.top_k, C, o.codec_offset, L, d_seed};
  SampleParams sp_all = sp;
  sp_all.noise = noise_;
  SampleParams sp_rest = sp_all;
  sp_rest.noise_frames = o.num_frames;  // one stream: noise row (frame * L + level)
  const char* head0 = static_cast<const char*>(m.lm_head) + static_cast<size_t>(o.codec_offset) * D * esz();
  const int ns = spec_count(o);
  for (int f = 0; f < o.num_frames; ++f) {
    if (f >= ns) {  // past the speculated frames: the plain decode
      enqueue_plain_frame(o, f, sp);
      continue;
    }
    int* tok = d_tokens + static_cast<size_t>(f) * L;
    launch_temporal_p(t_in, f, t_out);
    if (o.record_temporal) copy(static_cast<char*>(o.record_temporal) + f * row_bytes, t_out, row_bytes);
    // verification pass: rows 2i + r
    spec_inputs(dt, t_out, m.emb, d_drafts_ + static_cast<size_t>(f) * L, L, D, sx_, stream);
    for (int i = 0; i < c.num_depth_layers; ++i) {
      const DecoderLayerW& W = m.dep[i];
      rmsnorm_rows(dt, sx_, W.norm_sa, 1e-6f, R2, D, sxn_, stream);
      bgemm_qkv_pos(sxn_, R2, D, W.wqkv, HD, sq_, dk(i), dv(i), H, L, rows, stream);
      self_attn_at(dt, R2, sq_, dk(i), dv(i), H, L, 0, 0, nullptr, m.dbias, m.dbuckets, satt_, stream, rows);
      bgemm_resid(satt_, R2, HD, W.wo, D, sx_, D, stream);
      rmsnorm_rows(dt, sx_, W.norm_ff, 1e-6f, R2, D, sxn_, stream);
      bgemm_geglu(sxn_, R2, D, W.w01, FF, sffh_, FF, stream);
      bgemm_resid(sffh_, R2, FF, W.wo2, D, sx_, D, stream);
    }
    rmsnorm_rows(dt, sx_, m.dec_norm, 1e-6f, R2, D, sxn_, stream);
    bgemm_f32_grouped(sxn_, rows, D, head0, static_cast<long>(C) * D, C, slog_, C, L, stream);
    draw_levels(slog_, sp_all, f, L, sdrawn_, stream);
    int* decided = sdecided_ + f;
    sp_rest.decided = decided;
    spec_accept(dt, sdrawn_, d_drafts_ + static_cast<size_t>(f) * L, L, tok, decided, m.emb, D, d_in, stream);
    float* rec = o.record_slices ? o.record_slices + static_cast<size_t>(f) * L * rows * C : nullptr;
    if (lds_l_ > 0) {
      // the levels after the first disagreement in one persistent launch; the
      // decided levels' logits come from the verification pass
      if (rec)
        for (int l = 0; l < L; ++l) spec_record(slog_, nullptr, decided, l, C, rec + static_cast<size_t>(l) * rows * C, stream);
      FrameArgs fa{};
      fa.d = depth_args(nullptr, 0, head0, C, nullptr, nullptr);
      fa.d.sp = sp;
      fa.d.sp.decided = decided;
      fa.d.frame = f;
      fa.d.tokens = d_tokens;
      fa.d.emb = m.emb;
      fa.d.noise = noise_ + static_cast<size_t>(f) * L * C;
      fa.codebook = C;
      fa.levels = L;
      fa.rec_slices = rec;
      fa.qkv_table = qkv_table_;
      launch_levels(dt, fa, persist_grid_, lds_l_, stream);
      frame_mean_tokens(dt, tok, L, m.emb, D, t_in, stream);
      continue;
    }
    if (rec) spec_record(slog_, slice, decided, 0, C, rec, stream);
    // the levels after the first disagreement; a decided level's step and
    // draw return at once, its draw feeding the known token on
    for (int l = 1; l < L; ++l) {
      const char* head = head0 + static_cast<size_t>(C) * l * D * esz();
      StepArgs a = depth_args(d_in, l, head, C, slice, nullptr);
      a.sp = sp_rest;
      launch_step(dt, a, persist_grid_, lds_d_, stream);
      sample_level(dt, slice, sp_rest, f, l, f * L + l, nullptr, d_tokens, nullptr, m.emb, D, d_in, fsum, sfm_,
                   stream);
      if (rec) spec_record(slog_, slice, decided, l, C, rec + static_cast<size_t>(l) * rows * C, stream);
    }
    frame_mean_tokens(dt, tok, L, m.emb, D, t_in, stream);
  }
}

void State::check_device_error() {
  if (!persistent()) return;
  MRT_HIP_CHECK(hipMemcpyAsync(h_err_, ll_bufs().err, sizeof(int), hipMemcpyDeviceToHost, stream));
  MRT_HIP_CHECK(hipStreamSynchronize(stream));
  if (*h_err_ != 0) {
    *h_err_ = 0;
    reset_handoff();
    throw Error(3, "a hand-off poll timed out in a persistent step kernel (results discarded)");
  }
}

State::~State() {
  (void)hipSetDevice(m.device);
  if (stream) (void)hipStreamSynchronize(stream);
  for (DecodeGraph& g : graphs_) {
    (void)hipGraphExecDestroy(g.exec);
    (void)hipGraphDestroy(g.graph);
  }
  for (hipEvent_t e : ev_dec_)
    if (e) (void)hipEventDestroy(e);
  for (hipEvent_t e : ev_enc_)
    if (e) (void)hipEventDestroy(e);
  if (h_prof_) (void)hipHostFree(h_prof_);
  for (void* p : allocs_) (void)hipFree(p);
  if (h_pinned) (void)hipHostFree(h_pinned);
  if (h_err_) (void)hipHostFree(h_err_);
  if (h_seed_) (void)hipHostFree(h_seed_);
  if (stream) (void)hipStreamDestroy(stream);
}

char* State::tk(int i) const {
  const size_t n = static_cast<size_t>(rows) * m.cfg.num_heads * F * 64 * esz();
  return static_cast<char*>(tkv) + (2 * i) * n;
}
char* State::tv(int i) const {
  const size_t n = static_cast<size_t>(rows) * m.cfg.num_heads * F * 64 * esz();
  return static_cast<char*>(tkv) + (2 * i + 1) * n;
}
char* State::dk(int i) const {
  const size_t n = static_cast<size_t>(rows) * m.cfg.num_heads * m.cfg.rvq_depth * 64 * esz();
  return static_cast<char*>(dkv) + (2 * i) * n;
}
char* State::dv(int i) const {
  const size_t n = static_cast<size_t>(rows) * m.cfg.num_heads * m.cfg.rvq_depth * 64 * esz();
  return static_cast<char*>(dkv) + (2 * i + 1) * n;
}
char* State::ck(int i) const {
  const size_t n = static_cast<size_t>(rows) * m.cfg.num_heads * S * 64 * esz();
  return static_cast<char*>(cross) + (2 * i) * n;
}
char* State::cv(int i) const {
  const size_t n = static_cast<size_t>(rows) * m.cfg.num_heads * S * 64 * esz();
  return static_cast<char*>(cross) + (2 * i + 1) * n;
}

void State::copy(void* dst, const void* src, size_t bytes) { copy_dev(dst, src, bytes, stream); }

void State::sync() {
  MRT_HIP_CHECK(hipStreamSynchronize(stream));
  check_device_error();
}

// Depthformer::encode (model.cpp:226-241) followed by the cross K/V projection
// of every temporal layer (modules.cpp:448-455).
void State::encode(const int32_t* tokens_host) {
  const Config& c = m.cfg;
  const int M = rows * S;
  for (int i = 0; i < M; ++i)
    MRT_REQUIRE(tokens_host[i] >= 0 && tokens_host[i] < c.vocab_size, "encode: token id out of range");
  MRT_HIP_CHECK(hipSetDevice(m.device));
  MRT_HIP_CHECK(hipStreamSynchronize(stream));  // staging buffer reuse
  std::memcpy(h_pinned, tokens_host, static_cast<size_t>(M) * 4);
  MRT_HIP_CHECK(hipMemcpyAsync(d_enc_tok, h_pinned, static_cast<size_t>(M) * 4, hipMemcpyHostToDevice, stream));
  encode_device();
}

void run_encoder(const Model& m, const EncoderBufs& b, hipStream_t s) {
  const Config& c = m.cfg;
  const int M = b.rows * b.S;
  const DType dt = m.dt;
  const int D = c.d_model, HD = c.hd(), FF = c.d_ff, H = c.num_heads;
  encoder_embed(dt, m.emb, m.pe, b.tok, M, b.S, D, b.ex, s);
  for (const auto& L : m.enc) {
    rmsnorm_rows(dt, b.ex, L.norm_attn, 1e-6f, M, D, b.exn, s);
    gemm(dt, b.exn, L.wqkv, M, 3 * HD, D, {GemmEpi::Store, b.eqkv}, s);
    encoder_attn(dt, b.eqkv, b.rows, b.S, H, b.eattn, s);
    gemm(dt, b.eattn, L.wo, M, D, HD, {GemmEpi::Resid, b.ex}, s);
    rmsnorm_rows(dt, b.ex, L.norm_ff, 1e-6f, M, D, b.exn, s);
    gemm(dt, b.exn, L.w01, M, 2 * FF, D, {GemmEpi::Geglu, b.effh}, s);
    gemm(dt, b.effh, L.wo2, M, D, FF, {GemmEpi::Resid, b.ex}, s);
  }
  rmsnorm_rows(dt, b.ex, m.enc_norm, 1e-6f, M, D, b.enc_out, s);
  project_cross_kv(m, b.enc_out, b.rows, b.S, b.cross, s);
}

void project_cross_kv(const Model& m, const void* enc_out, int rows, int S, void* cross, hipStream_t s) {
  const Config& c = m.cfg;
  if (c.num_temporal_layers == 0) return;
  GemmEpiArgs e;
  e.kind = GemmEpi::CrossKV;
  e.C = cross;
  e.nb = rows;
  e.H = c.num_heads;
  e.S = S;
  e.HD = c.hd();
  gemm(m.dt, enc_out, m.wkv_cross, rows * S, c.num_temporal_layers * 2 * c.hd(), c.d_model, e, s);
}

// The encoder on the token ids already in d_enc_tok (range-checked by whoever
// wrote them), then the cross K/V of every temporal layer.
void State::encode_device() {
  MRT_HIP_CHECK(hipSetDevice(m.device));
  EncoderBufs b;
  b.rows = rows;
  b.S = S;
  b.tok = d_enc_tok;
  b.ex = ex;
  b.exn = exn;
  b.eqkv = eqkv;
  b.eattn = eattn;
  b.effh = effh;
  b.enc_out = enc_out;
  b.cross = cross;
  if (!ev_enc_[0]) {
    MRT_HIP_CHECK(hipEventCreate(&ev_enc_[0]));
    MRT_HIP_CHECK(hipEventCreate(&ev_enc_[1]));
  }
  MRT_HIP_CHECK(hipEventRecord(ev_enc_[0], stream));
  run_encoder(m, b, stream);
  MRT_HIP_CHECK(hipEventRecord(ev_enc_[1], stream));
  enc_timed_ = true;
  cross_ready_ = true;
}

void State::project_cross(const void* src) {
  project_cross_kv(m, src, rows, S, cross, stream);
  cross_ready_ = true;
}

// One temporal step on the device (model.cpp:493-513 eager semantics).
void State::run_temporal(const void* in, int f, void* out, const void* bias) {
  const Config& c = m.cfg;
  const DType dt = m.dt;
  const int D = c.d_model, HD = c.hd(), FF = c.d_ff, H = c.num_heads;
  copy(out, in, static_cast<size_t>(rows) * D * esz());
  for (int i = 0; i < c.num_temporal_layers; ++i) {
    const DecoderLayerW& L = m.tmp[i];
    gemv_qkv(dt, rows, L.wqkv, HD, D, out, D, {L.norm_sa}, q, tk(i), tv(i), H, F, f, stream);
    self_attn(dt, rows, q, tk(i), tv(i), H, F, f + 1, f, m.tbias, m.tbuckets, attn, stream, bias);
    gemv_resid(dt, rows, L.wo, D, HD, attn, HD, {}, out, D, stream);
    gemv_store(dt, rows, L.wq_c, HD, D, out, D, {L.norm_ca}, q, HD, stream);
    cross_attn(dt, rows, q, ck(i), cv(i), H, S, attn, part, nsplit, stream);
    gemv_resid(dt, rows, L.wo_c, D, HD, attn, HD, {}, out, D, stream);
    gemv_geglu(dt, rows, L.w01, FF, D, out, D, {L.norm_ff}, ffh, FF, stream);
    gemv_resid(dt, rows, L.wo2, D, FF, ffh, FF, {}, out, D, stream);
  }
}

// One depth step on the device (model.cpp:638-658): 4 layers, decoder_norm,
// lm_head (full vocabulary or one level's rows).
// Depthformer::depth_forward_full (model.cpp:243-268): the depth stack over k
// positions of both rows in one pass (rows m = b*k + i), causal unless asked
// otherwise, with the rel-pos bias of the k x k block or an explicit
// (H, k, k) one, then decoder_norm and lm_head over the whole vocabulary.
// The caches are not touched (the reference discards the pass's K/V).
void State::depth_forward_full(const void* emb, int k, const void* bias, bool causal, float* logits) {
  const Config& c = m.cfg;
  const DType dt = m.dt;
  MRT_REQUIRE(k >= 1 && k <= c.rvq_depth, "depth_forward_full: k_len must be in [1, rvq_depth]");
  const int D = c.d_model, HD = c.hd(), FF = c.d_ff, H = c.num_heads, M = rows * k;
  MRT_HIP_CHECK(hipSetDevice(m.device));
  copy(sx_, emb, static_cast<size_t>(M) * D * esz());
  auto gemm_to = [&](const void* A, const void* W, int N, int K, GemmEpi kind, void* C) {
    GemmEpiArgs e;
    e.kind = kind;
    e.C = C;
    gemm(dt, A, W, M, N, K, e, stream);
  };
  for (int i = 0; i < c.num_depth_layers; ++i) {
    const DecoderLayerW& W = m.dep[i];
    rmsnorm_rows(dt, sx_, W.norm_sa, 1e-6f, M, D, sxn_, stream);
    gemm_to(sxn_, W.wqkv, 3 * HD, D, GemmEpi::Store, sqkv_);
    full_attn(dt, rows, k, H, sqkv_, bias, m.dbias, m.dbuckets, causal, satt_, stream);
    gemm_to(satt_, W.wo, D, HD, GemmEpi::Resid, sx_);
    rmsnorm_rows(dt, sx_, W.norm_ff, 1e-6f, M, D, sxn_, stream);
    gemm_to(sxn_, W.w01, 2 * FF, D, GemmEpi::Geglu, sffh_);
    gemm_to(sffh_, W.wo2, D, FF, GemmEpi::Resid, sx_);
  }
  rmsnorm_rows(dt, sx_, m.dec_norm, 1e-6f, M, D, sxn_, stream);
  gemm_to(sxn_, m.lm_head, c.vocab_size, D, GemmEpi::StoreF32, logits);
  MRT_HIP_CHECK(hipStreamSynchronize(stream));
}

void State::run_depth(const void* in, int l, int level, int C, int off, float* logits, const void* bias) {
  const Config& c = m.cfg;
  const DType dt = m.dt;
  const int D = c.d_model, HD = c.hd(), FF = c.d_ff, H = c.num_heads, L = c.rvq_depth;
  copy(x, in, static_cast<size_t>(rows) * D * esz());
  for (int i = 0; i < c.num_depth_layers; ++i) {
    const DecoderLayerW& W = m.dep[i];
    gemv_qkv(dt, rows, W.wqkv, HD, D, x, D, {W.norm_sa}, q, dk(i), dv(i), H, L, l, stream);
    self_attn(dt, rows, q, dk(i), dv(i), H, L, l + 1, l, m.dbias, m.dbuckets, attn, stream, bias);
    gemv_resid(dt, rows, W.wo, D, HD, attn, HD, {}, x, D, stream);
    gemv_geglu(dt, rows, W.w01, FF, D, x, D, {W.norm_ff}, ffh, FF, stream);
    gemv_resid(dt, rows, W.wo2, D, FF, ffh, FF, {}, x, D, stream);
  }
  if (level >= 0) {
    const char* rows0 = static_cast<const char*>(m.lm_head) + static_cast<size_t>(off + C * level) * D * esz();
    gemv_f32(dt, rows, rows0, C, D, x, D, {m.dec_norm}, logits, C, stream);
  } else {
    gemv_f32(dt, rows, m.lm_head, c.vocab_size, D, x, D, {m.dec_norm}, logits, c.vocab_size, stream);
  }
}

void State::temporal_step(const void* in, const void* enc, int f, void* out, const void* bias) {
  MRT_REQUIRE(f >= 0 && f < F, "temporal_step: frame_idx out of range for this state");
  MRT_HIP_CHECK(hipSetDevice(m.device));
  if (f == 0) {
    temporal_len_ = 0;
    if (enc != nullptr) project_cross(enc);
  }
  if (!cross_ready_)
    throw Error(2, "temporal_step: cross-attention K/V not populated (call encode or pass enc_out at frame 0)");
  if (temporal_len_ != f)
    throw Error(1, "temporal_step: cache holds " + std::to_string(temporal_len_) + " entries, frame_idx " +
                       std::to_string(f));
  if (persistent()) {
    reserve_epochs(1);
    PersistSection gate(m.device, stream);
    launch_temporal_p(in, f, out, bias);
  } else {
    run_temporal(in, f, out, bias);
  }
  temporal_len_ = f + 1;
}

void State::depth_step(const void* in, int l, int level, int C, int off, float* logits, const void* bias) {
  const Config& c = m.cfg;
  MRT_REQUIRE(l >= 0 && l < c.rvq_depth, "depth_step: depth_idx out of range");
  if (level >= 0) {
    MRT_REQUIRE(C >= 1 && off >= 0 && off + C * (level + 1) <= c.vocab_size,
                "depth_step: level slice outside the vocabulary");
  }
  MRT_HIP_CHECK(hipSetDevice(m.device));
  if (l == 0) depth_len_ = 0;
  if (depth_len_ != l)
    throw Error(1, "depth_step: cache holds " + std::to_string(depth_len_) + " entries, depth_idx " +
                       std::to_string(l));
  if (persistent()) {
    const int D = c.d_model;
    const void* head = level >= 0
                           ? static_cast<const char*>(m.lm_head) + static_cast<size_t>(off + C * level) * D * esz()
                           : m.lm_head;
    reserve_epochs(1);
    PersistSection gate(m.device, stream);
    launch_depth_p(in, l, head, level >= 0 ? C : c.vocab_size, logits, nullptr, bias);
  } else {
    run_depth(in, l, level, C, off, logits, bias);
  }
  depth_len_ = l + 1;
}

void State::reset_cache(int kind) {
  MRT_REQUIRE(kind == 0 || kind == 1, "reset_cache: kind must be 0 (temporal) or 1 (depth)");
  if (kind == 0)
    temporal_len_ = 0;
  else
    depth_len_ = 0;
}

const void* Model::depth_qkv_table(int codebook, int offset, hipStream_t s) {
  const int L = cfg.rvq_depth, D = cfg.d_model, HD = cfg.hd();
  if (L < 2 || cfg.num_depth_layers < 1) return nullptr;
  MRT_REQUIRE(codebook >= 1 && offset >= 0 && offset + codebook * L <= cfg.vocab_size,
              "depth q/k/v table: codec levels exceed the vocabulary");
  std::lock_guard<std::mutex> lock(qkv_mu_);
  for (const QkvTable& t : qkv_tables_)
    if (t.codebook == codebook && t.offset == offset) return t.rows;
  // Tables are never evicted (a captured decode graph holds its table's
  // address); past the cap the decode computes layer 0 instead.
  if (qkv_tables_.size() >= kMaxQkvTables) return nullptr;
  MRT_HIP_CHECK(hipSetDevice(device));
  // Row r = (l - 1) * codebook + c is the token offset + codebook (l - 1) + c =
  // offset + r: the rows' inputs are the embedding rows offset .. offset + rows,
  // normalised in chunks through a workspace the model keeps.
  const int rows = (L - 1) * codebook;
  if (qkv_ws_ == nullptr) {
    MRT_HIP_CHECK(hipMalloc(&qkv_ws_, static_cast<size_t>(kQkvChunkRows) * D * esz));
    allocs_.push_back(qkv_ws_);
  }
  void* out = nullptr;
  MRT_HIP_CHECK(hipMalloc(&out, static_cast<size_t>(rows) * 3 * HD * esz));
  allocs_.push_back(out);
  for (int r0 = 0; r0 < rows; r0 += kQkvChunkRows) {
    const int n = std::min(kQkvChunkRows, rows - r0);
    const char* x = static_cast<const char*>(emb) + (static_cast<size_t>(offset) + r0) * D * esz;
    rmsnorm_rows(dt, x, dep[0].norm_sa, 1e-6f, n, D, qkv_ws_, s);
    GemmEpiArgs e;
    e.kind = GemmEpi::Store;
    e.C = static_cast<char*>(out) + static_cast<size_t>(r0) * 3 * HD * esz;
    gemm(dt, qkv_ws_, dep[0].wqkv, n, 3 * HD, D, e, s);
  }
  MRT_HIP_CHECK(hipStreamSynchronize(s));
  qkv_tables_.push_back(QkvTable{codebook, offset, out});
  return out;
}

void Model::precompute_biases(int kind, int n, void* out) const {
  MRT_REQUIRE(kind == 0 || kind == 1, "precompute_biases: kind must be 0 (temporal) or 1 (depth)");
  MRT_REQUIRE(n >= 1 && n < kBucketTable, "precompute_biases: n out of range");
  MRT_HIP_CHECK(hipSetDevice(device));
  hipStream_t s = nullptr;
  MRT_HIP_CHECK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
  try {
    bias_rows(dt, kind == 0 ? tbias : dbias, kind == 0 ? tbuckets : dbuckets, cfg.num_heads, n, out, s);
    MRT_HIP_CHECK(hipStreamSynchronize(s));
  } catch (...) {
    (void)hipStreamDestroy(s);
    throw;
  }
  MRT_HIP_CHECK(hipStreamDestroy(s));
}

void State::enqueue_decode(const GenOpts& o) {
  const Config& c = m.cfg;
  const DType dt = m.dt;
  const int D = c.d_model;
  SampleParams sp{o.guidance_weight, o.temperature, o.top_k, o.codebook, o.codec_offset, o.rvq_depth, d_seed};
  // Frame 0 feeds emb(PAD = 0) on both rows (decode.cpp:339-341, 366-368).
  embed_fill(dt, m.emb, D, 0, rows, t_in, stream);
  const size_t row_bytes = static_cast<size_t>(rows) * D * esz();
  for (int f = 0; f < o.num_frames; ++f) {
    run_temporal(t_in, f, t_out);
    if (o.record_temporal)
      copy(static_cast<char*>(o.record_temporal) + f * row_bytes, t_out, row_bytes);
    for (int l = 0; l < o.rvq_depth; ++l) {
      run_depth(l == 0 ? t_out : d_in, l, l, o.codebook, o.codec_offset, slice);
      if (o.record_slices)
        copy(o.record_slices + (static_cast<size_t>(f) * o.rvq_depth + l) * rows * o.codebook, slice,
             static_cast<size_t>(rows) * o.codebook * 4);
      sample_level(dt, slice, sp, f, l, f * o.rvq_depth + l, o.teacher ? d_teacher : nullptr, d_tokens,
                   o.record_drawn, m.emb, D, d_in, fsum, t_in, stream);
    }
    if (o.record_frame_mean)
      copy(static_cast<char*>(o.record_frame_mean) + f * row_bytes, t_in, row_bytes);
  }
}

void Model::sample_noalloc(const float* slice_dev, const GenOpts& o, int frame, int level, int32_t* token_dev,
                           hipStream_t stream) const {
  MRT_REQUIRE(o.codebook >= 1 && o.codebook <= 1024, "sample: codebook_size must be in [1, 1024]");
  MRT_REQUIRE(level >= 0 && level < o.rvq_depth && frame >= 0, "sample: frame/level out of range");
  MRT_REQUIRE(o.codec_offset >= 0 && o.codec_offset + o.codebook * o.rvq_depth <= cfg.vocab_size,
              "sample: codec levels exceed the vocabulary");
  MRT_REQUIRE(o.temperature >= 0.0f, "sample: temperature must be >= 0");
  MRT_HIP_CHECK(hipSetDevice(device));
  SampleParams sp{o.guidance_weight, o.temperature, o.top_k, o.codebook, o.codec_offset, o.rvq_depth, nullptr};
  sample_level_noalloc(dt, device, emb, cfg.d_model, slice_dev, sp, o.seed, frame, level, token_dev, stream);
}

int State::sample(const float* slice_dev, const GenOpts& o, int frame, int level) {
  const Config& c = m.cfg;
  MRT_REQUIRE(o.codebook >= 1 && o.codebook <= 1024, "sample: codebook_size must be in [1, 1024]");
  MRT_REQUIRE(level >= 0 && level < o.rvq_depth && frame >= 0, "sample: frame/level out of range");
  MRT_REQUIRE(o.codec_offset >= 0 && o.codec_offset + o.codebook * o.rvq_depth <= c.vocab_size,
              "sample: codec levels exceed the vocabulary");
  MRT_REQUIRE(o.temperature >= 0.0f, "sample: temperature must be >= 0");
  MRT_HIP_CHECK(hipSetDevice(m.device));
  *h_seed_ = o.seed;  // its previous copy ended before the last call returned
  MRT_HIP_CHECK(hipMemcpyAsync(d_seed, h_seed_, 8, hipMemcpyHostToDevice, stream));
  SampleParams sp{o.guidance_weight, o.temperature, o.top_k, o.codebook, o.codec_offset, o.rvq_depth, d_seed};
  // Token goes to slot 0 of the token buffer; the feedback outputs land in
  // scratch rows that the next decode overwrites.
  prev_frames_ = 0;  // slot 0 of the token buffer is no longer the last call's
  sample_level(m.dt, slice_dev, sp, frame, level, 0, nullptr, d_tokens, nullptr, m.emb, c.d_model, d_in, fsum,
               x, stream);
  MRT_HIP_CHECK(hipMemcpyAsync(h_pinned, d_tokens, 4, hipMemcpyDeviceToHost, stream));
  MRT_HIP_CHECK(hipStreamSynchronize(stream));
  return h_pinned[0];
}

void State::enqueue_decode_any(const GenOpts& o) {
  if (spec_drafts_)
    enqueue_decode_spec(o);
  else if (persistent())
    enqueue_decode_p(o);
  else
    enqueue_decode(o);
}

// The captured decode loop for these options: replayed when a graph with the
// same key exists, else captured (and the least recently used graph dropped
// once kMaxDecodeGraphs are held).
hipGraphExec_t State::decode_graph(const GenOpts& o) {
  const std::vector<double> key = {
      (double)o.num_frames, (double)o.rvq_depth, (double)o.temperature, (double)o.top_k,
      (double)o.guidance_weight, (double)o.codebook, (double)o.codec_offset, o.teacher ? 1.0 : 0.0,
      spec_drafts_ ? 1.0 : 0.0, (double)spec_count(o), profile_ ? 1.0 : 0.0,
      (double)reinterpret_cast<uintptr_t>(o.record_slices),
      (double)reinterpret_cast<uintptr_t>(o.record_temporal),
      (double)reinterpret_cast<uintptr_t>(o.record_drawn),
      (double)reinterpret_cast<uintptr_t>(o.record_frame_mean)};
  for (DecodeGraph& g : graphs_)
    if (g.key == key) {
      g.used = ++graph_clock_;
      return g.exec;
    }
  if (graphs_.size() >= kMaxDecodeGraphs) {
    auto lru = std::min_element(graphs_.begin(), graphs_.end(),
                                [](const DecodeGraph& a, const DecodeGraph& b) { return a.used < b.used; });
    MRT_HIP_CHECK(hipStreamSynchronize(stream));  // its last replay has ended
    (void)hipGraphExecDestroy(lru->exec);
    (void)hipGraphDestroy(lru->graph);
    graphs_.erase(lru);
  }
  MRT_HIP_CHECK(hipStreamSynchronize(stream));  // capture starts on an idle stream
  MRT_HIP_CHECK(hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal));
  hipGraph_t graph = nullptr;
  try {
    enqueue_decode_any(o);
  } catch (...) {
    (void)hipStreamEndCapture(stream, &graph);
    if (graph) (void)hipGraphDestroy(graph);
    throw;
  }
  MRT_HIP_CHECK(hipStreamEndCapture(stream, &graph));
  hipGraphExec_t exec = nullptr;
  const hipError_t e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
  if (e != hipSuccess) {
    (void)hipGraphDestroy(graph);
    MRT_HIP_CHECK(e);
  }
  graphs_.push_back(DecodeGraph{key, graph, exec, ++graph_clock_});
  return exec;
}

void State::generate(const int32_t* enc_tokens_host, const GenOpts& o, int32_t* out_host) {
  const Config& c = m.cfg;
  MRT_REQUIRE(o.num_frames >= 1 && o.num_frames <= F, "generate: num_frames exceeds the state's max_frames");
  MRT_REQUIRE(o.rvq_depth == c.rvq_depth, "generate: rvq_depth must equal the model's rvq_depth");
  MRT_REQUIRE(o.codebook >= 1 && o.codebook <= 1024, "generate: codebook_size must be in [1, 1024]");
  MRT_REQUIRE(o.codec_offset >= 0 && o.codec_offset + o.codebook * o.rvq_depth <= c.vocab_size,
              "generate: codec levels exceed the vocabulary");
  MRT_REQUIRE(o.temperature >= 0.0f, "generate: temperature must be >= 0");
  MRT_HIP_CHECK(hipSetDevice(m.device));
  if (enc_tokens_host) encode(enc_tokens_host);
  if (!cross_ready_) throw Error(2, "generate: no encoder output (pass enc_tokens or call encode)");
  const size_t nt = static_cast<size_t>(o.num_frames) * o.rvq_depth;
  // No wait on the stream here unless the staging buffer is needed: work
  // already enqueued (an encoder) runs on while the decode is enqueued.
  if (o.teacher) {
    for (size_t i = 0; i < nt; ++i)
      MRT_REQUIRE(o.teacher[i] >= 0 && o.teacher[i] < c.vocab_size, "generate: teacher id out of range");
    MRT_HIP_CHECK(hipStreamSynchronize(stream));  // staging reuse (an encode may be reading it)
    std::memcpy(h_pinned, o.teacher, nt * 4);
    MRT_HIP_CHECK(hipMemcpyAsync(d_teacher, h_pinned, nt * 4, hipMemcpyHostToDevice, stream));
  }
  *h_seed_ = o.seed;  // its previous copy ended before the last call returned
  MRT_HIP_CHECK(hipMemcpyAsync(d_seed, h_seed_, 8, hipMemcpyHostToDevice, stream));
  // Speculative decoding drafts frame f with the previous call's tokens of
  // frame f (build_depth_draft, decode.cpp:150-166): copied before this call
  // overwrites them.  Without a previous call of the same length it does not
  // speculate (as the reference's first chunk).
  spec_drafts_ = speculating(o) && prev_frames_ == o.num_frames;
  if (spec_drafts_) copy(d_drafts_, d_tokens, nt * 4);

  if (persistent()) reserve_epochs(decode_launches(o));
  if (!ev_dec_[0]) {
    MRT_HIP_CHECK(hipEventCreate(&ev_dec_[0]));
    MRT_HIP_CHECK(hipEventCreate(&ev_dec_[1]));
  }
  dec_launches_ = persistent() ? decode_launches(o) : 0;
  // built once per (codebook, offset) before any capture; waits for the stream then
  qkv_table_ = frame_kernel_ && qkv_table_on_ ? m.depth_qkv_table(o.codebook, o.codec_offset, stream) : nullptr;
  hipGraphExec_t exec = o.use_graph ? decode_graph(o) : nullptr;
  {
    // persistent grids of other states on this device run before or after
    // this decode, never beside it
    std::optional<PersistSection> gate;
    if (persistent()) gate.emplace(m.device, stream);
    MRT_HIP_CHECK(hipEventRecord(ev_dec_[0], stream));
    if (exec)
      MRT_HIP_CHECK(hipGraphLaunch(exec, stream));
    else
      enqueue_decode_any(o);
    MRT_HIP_CHECK(hipEventRecord(ev_dec_[1], stream));
  }
  dec_timed_ = true;
  // the frame kernel's phase stamps (the speculative path runs per-step launches)
  prof_frames_ = profile_ && persistent() && frame_kernel_ && !spec_drafts_ ? o.num_frames : 0;
  if (prof_frames_ > 0)
    MRT_HIP_CHECK(hipMemcpyAsync(h_prof_, d_prof_, static_cast<size_t>(prof_frames_) * 4 * sizeof(uint64_t),
                                 hipMemcpyDeviceToHost, stream));
  MRT_HIP_CHECK(hipMemcpyAsync(h_pinned, d_tokens, nt * 4, hipMemcpyDeviceToHost, stream));
  const int nspec = spec_count(o);
  if (nspec > 0)
    MRT_HIP_CHECK(hipMemcpyAsync(h_pinned + nt, sdecided_, static_cast<size_t>(nspec) * 4, hipMemcpyDeviceToHost,
                                 stream));
  MRT_HIP_CHECK(hipStreamSynchronize(stream));
  check_device_error();
  print_trace();
  std::memcpy(out_host, h_pinned, nt * 4);
  spec_acc_ = -1.f;
  if (nspec > 0) {  // levels 0..n of frame f came from the verification pass (n = L: all)
    long from_pass = 0;
    for (int f = 0; f < nspec; ++f) from_pass += std::min(h_pinned[nt + f] + 1, o.rvq_depth);
    spec_acc_ = static_cast<float>(from_pass) / static_cast<float>(static_cast<long>(nspec) * o.rvq_depth);
  }
  temporal_len_ = o.num_frames;
  depth_len_ = o.rvq_depth;
  prev_frames_ = o.num_frames;
}

float State::last_decode_ms(int* launches) {
  if (!dec_timed_) throw Error(1, "decode time: no generate call on this state yet");
  MRT_HIP_CHECK(hipEventSynchronize(ev_dec_[1]));
  float ms = 0.f;
  MRT_HIP_CHECK(hipEventElapsedTime(&ms, ev_dec_[0], ev_dec_[1]));
  if (launches) *launches = dec_launches_;
  return ms;
}

State::DecodeProfile State::decode_profile() {
  DecodeProfile r;
  int launches = 0;
  r.total_ms = last_decode_ms(&launches);
  if (enc_timed_) {
    MRT_HIP_CHECK(hipEventSynchronize(ev_enc_[1]));
    MRT_HIP_CHECK(hipEventElapsedTime(&r.encoder_ms, ev_enc_[0], ev_enc_[1]));
  }
  r.frames = prof_frames_;
  if (prof_frames_ > 0) {
    int khz = 0;
    MRT_HIP_CHECK(hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, m.device));
    MRT_REQUIRE(khz > 0, "decode profile: the device reports no wall-clock rate");
    double t = 0, d = 0, w = 0;
    for (int f = 0; f < prof_frames_; ++f) {
      const uint64_t* q = h_prof_ + 4 * f;
      t += static_cast<double>(q[1] - q[0]);
      d += static_cast<double>(q[2] - q[1]) - static_cast<double>(q[3]);
      w += static_cast<double>(q[3]);
    }
    const double ms = 1.0 / khz;  // one tick in ms
    r.temporal_ms = static_cast<float>(t * ms);
    r.depth_ms = static_cast<float>(d * ms);
    r.sample_ms = static_cast<float>(w * ms);
  }
  return r;
}

void State::compile(const GenOpts& o) {
  MRT_HIP_CHECK(hipSetDevice(m.device));
  const bool had_cross = cross_ready_;
  const int tl = temporal_len_, dl = depth_len_;
  if (!had_cross) {  // an encoding of PAD ids, dropped afterwards
    MRT_HIP_CHECK(hipMemsetAsync(d_enc_tok, 0, static_cast<size_t>(rows) * S * sizeof(int), stream));
    encode_device();
  }
  GenOpts g = o;
  g.teacher = nullptr;
  g.record_slices = nullptr;
  g.record_temporal = nullptr;
  g.record_drawn = nullptr;
  g.record_frame_mean = nullptr;
  std::vector<int32_t> tmp(static_cast<size_t>(std::max(o.num_frames, 1)) * std::max(o.rvq_depth, 1));
  prev_frames_ = 0;
  generate(nullptr, g, tmp.data());
  if (g.speculative && speculating(g)) generate(nullptr, g, tmp.data());  // the speculative graph too
  cross_ready_ = had_cross;
  temporal_len_ = tl;
  depth_len_ = dl;
  prev_frames_ = 0;  // the dry run's tokens are no drafts
  spec_acc_ = -1.f;
  dec_timed_ = false;
  enc_timed_ = false;
  prof_frames_ = 0;
}

float State::phase_trace(uint64_t* out, int n) {
  MRT_REQUIRE(d_trace_ != nullptr, "phase trace: the state was created without MRT_TRACE_PHASES");
  MRT_REQUIRE(n >= 2 * kTraceSlots, "phase trace: the output holds fewer than 2 x 512 words");
  MRT_HIP_CHECK(hipStreamSynchronize(stream));
  MRT_HIP_CHECK(hipMemcpy(out, d_trace_, 2 * kTraceSlots * sizeof(uint64_t), hipMemcpyDeviceToHost));
  int khz = 0;
  MRT_HIP_CHECK(hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, m.device));
  return static_cast<float>(khz) / 1000.f;
}

void* State::buffer(int which, int layer, size_t* bytes) {
  const Config& c = m.cfg;
  const size_t H = c.num_heads;
  auto chk = [&](int n) { MRT_REQUIRE(layer >= 0 && layer < n, "state buffer: layer out of range"); };
  switch (which) {
    case 0:
      *bytes = static_cast<size_t>(rows) * S * c.d_model * esz();
      return enc_out;
    case 1:
    case 2:
      chk(c.num_temporal_layers);
      *bytes = static_cast<size_t>(rows) * H * S * 64 * esz();
      return which == 1 ? ck(layer) : cv(layer);
    case 3:
    case 4:
      chk(c.num_temporal_layers);
      *bytes = static_cast<size_t>(rows) * H * F * 64 * esz();
      return which == 3 ? tk(layer) : tv(layer);
    case 5:
    case 6:
      chk(c.num_depth_layers);
      *bytes = static_cast<size_t>(rows) * H * c.rvq_depth * 64 * esz();
      return which == 5 ? dk(layer) : dv(layer);
    case 7:
      *bytes = static_cast<size_t>(rows) * S * 4;
      return d_enc_tok;
    default:
      throw Error(1, "state buffer: unknown buffer id");
  }
}

void State::set_cache_length(int kind, int length) {
  if (kind == 0) {
    MRT_REQUIRE(length >= 0 && length <= F, "set_cache_length: temporal length out of range");
    temporal_len_ = length;
  } else if (kind == 1) {
    MRT_REQUIRE(length >= 0 && length <= m.cfg.rvq_depth, "set_cache_length: depth length out of range");
    depth_len_ = length;
  } else if (kind == 2) {
    cross_ready_ = length != 0;
  } else {
    throw Error(1, "set_cache_length: kind must be 0 (temporal), 1 (depth) or 2 (cross ready)");
  }
}

}  // namespace mrt
