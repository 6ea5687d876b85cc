// Codec decode host side: weight packing, per-frame-count launch plans and
// the decode sequence (system.cpp:373-390: rvq_dequantization, the decoder,
// istft_postprocess).
#include "codec.hpp"

#include <algorithm>
#include <cmath>
#include <string>

namespace mrt {

namespace {

int round_up(int v, int m) { return (v + m - 1) / m * m; }

void check_shape(const HostTensor& t, const std::string& name, std::vector<int64_t> want) {
  if (t.shape != want) {
    std::string got, exp;
    for (auto d : t.shape) got += std::to_string(d) + ",";
    for (auto d : want) exp += std::to_string(d) + ",";
    throw Error(1, "codec: tensor " + name + " has shape (" + got + ") but (" + exp + ") is required");
  }
}

}  // namespace

float* Codec::dalloc(size_t floats) {
  void* d = nullptr;
  MRT_HIP_CHECK(hipMalloc(&d, std::max<size_t>(floats * 4, 256)));
  allocs_.push_back(d);
  return static_cast<float*>(d);
}

// WNConv2d (spectrostream.cpp:125-139): stored (O, I, kH, kW) -> one sub-problem
// with rows (t * I + c), t = kh * kW + kw, columns O padded to the tile width.
Codec::Conv Codec::pack_conv(const TensorSource& w, const std::string& name, int o, int i, int kh, int kw) {
  const HostTensor& t = w.tensor(name + ".weight");
  check_shape(t, name + ".weight", {o, i, kh, kw});
  const HostTensor& b = w.tensor(name + ".bias");
  check_shape(b, name + ".bias", {o});
  Conv c;
  c.cin = i;
  c.cout = o;
  c.cout_pad = round_up(o, 64);
  std::vector<float> h(static_cast<size_t>(kh) * kw * i * c.cout_pad, 0.f);
  for (int oo = 0; oo < o; ++oo)
    for (int ii = 0; ii < i; ++ii)
      for (int y = 0; y < kh; ++y)
        for (int x = 0; x < kw; ++x)
          h[(static_cast<size_t>(y * kw + x) * i + ii) * c.cout_pad + oo] =
              t.data[((static_cast<size_t>(oo) * i + ii) * kh + y) * kw + x];
  float* d = dalloc(h.size());
  MRT_HIP_CHECK(hipMemcpy(d, h.data(), h.size() * 4, hipMemcpyHostToDevice));
  c.w.push_back(d);
  c.bias = dalloc(o);
  MRT_HIP_CHECK(hipMemcpy(c.bias, b.data, o * 4, hipMemcpyHostToDevice));
  return c;
}

// WNConvTranspose2d (spectrostream.cpp:141-158): stored (I, O, kH, kW).  One
// sub-problem per output phase (ph, pw): taps (kh, kw) = (ph + sh j, pw + sw i),
// t = j * ni + i, reading input pixel (q_y - j, q_x - i).
Codec::Conv Codec::pack_transposed(const TensorSource& w, const std::string& name, int i, int o, int kh, int kw,
                                   int sh, int sw) {
  const HostTensor& t = w.tensor(name + ".weight");
  check_shape(t, name + ".weight", {i, o, kh, kw});
  const HostTensor& b = w.tensor(name + ".bias");
  check_shape(b, name + ".bias", {o});
  Conv c;
  c.cin = i;
  c.cout = o;
  c.cout_pad = round_up(o, 64);
  for (int ph = 0; ph < sh; ++ph)
    for (int pw = 0; pw < sw; ++pw) {
      const int nj = (kh - ph + sh - 1) / sh, ni = (kw - pw + sw - 1) / sw;
      std::vector<float> h(static_cast<size_t>(nj) * ni * i * c.cout_pad, 0.f);
      for (int j = 0; j < nj; ++j)
        for (int q = 0; q < ni; ++q) {
          const int y = ph + sh * j, x = pw + sw * q, tap = j * ni + q;
          for (int ii = 0; ii < i; ++ii)
            for (int oo = 0; oo < o; ++oo)
              h[(static_cast<size_t>(tap) * i + ii) * c.cout_pad + oo] =
                  t.data[((static_cast<size_t>(ii) * o + oo) * kh + y) * kw + x];
        }
      float* d = dalloc(h.size());
      MRT_HIP_CHECK(hipMemcpy(d, h.data(), h.size() * 4, hipMemcpyHostToDevice));
      c.w.push_back(d);
    }
  c.bias = dalloc(o);
  MRT_HIP_CHECK(hipMemcpy(c.bias, b.data, o * 4, hipMemcpyHostToDevice));
  return c;
}

Codec::Codec(const TensorSource& w, const TensorSource& cbs, const CodecConfig& c, int dev, int maxf)
    : cfg(c), device(dev), max_frames(maxf) {
  MRT_REQUIRE(max_frames >= 1 && max_frames <= 4096, "codec: max_frames must be in [1, 4096]");
  MRT_REQUIRE(cfg.blocks.size() == 7, "codec: the decoder has 7 blocks");
  MRT_REQUIRE(cfg.proj_ch % cfg.unfold == 0, "codec: proj channels must divide by the unfold factor");
  MRT_REQUIRE(cfg.n_fft == 2 * cfg.hop && cfg.hop % 16 == 0, "codec: n_fft must be 2 x hop");
  const int E = cfg.embedding_dim, P = cfg.proj_ch, C0 = P / cfg.unfold;
  auto ch_ok = [](int v) { return v >= 16 && v % 16 == 0; };
  MRT_REQUIRE(ch_ok(E) && ch_ok(P) && ch_ok(C0), "codec: channel counts must be multiples of 16");
  MRT_REQUIRE(cfg.blocks[0].in_ch == C0, "codec: block 0 input channels must equal proj / unfold");
  MRT_REQUIRE(cfg.blocks[0].out_ch % 32 == 0, "codec: block 0 output channels split into two stereo halves");
  for (size_t i = 0; i < cfg.blocks.size(); ++i) {
    const CodecBlockCfg& b = cfg.blocks[i];
    MRT_REQUIRE(ch_ok(b.in_ch) && ch_ok(b.out_ch), "codec: channel counts must be multiples of 16");
    MRT_REQUIRE(b.sh >= 1 && b.sw >= 1 && b.kth >= b.sh && b.ktw >= b.sw, "codec: kernel smaller than stride");
    MRT_REQUIRE(b.kph * b.kpw <= kConvMaxTaps && b.kth * b.ktw <= kConvMaxTaps, "codec: kernel too large");
    if (i >= 1) {
      const int prev = i == 1 ? cfg.blocks[0].out_ch / 2 : cfg.blocks[i - 1].out_ch;
      MRT_REQUIRE(b.in_ch == prev, "codec: block channel chain is inconsistent");
    }
  }
  MRT_REQUIRE(cfg.out_k * cfg.out_k <= kConvMaxTaps, "codec: output kernel too large");
  MRT_REQUIRE(cfg.out_ch == 2, "codec: the output conv gives (real, imag)");
  // every tensor present with its stored shape before any device work
  // (spectrostream.cpp:125-158, 163-262, 356-362)
  {
    auto conv = [&](const std::string& n, int o, int i, int kh, int kw) {
      check_shape(w.tensor(n + ".weight"), n + ".weight", {o, i, kh, kw});
      check_shape(w.tensor(n + ".bias"), n + ".bias", {o});
    };
    conv("input_proj.conv1", P, E, 1, 1);
    conv("input_proj.conv2", P, P, 1, 1);
    conv("input_proj.shortcut", P, E, 1, 1);
    conv("input_conv.conv1", C0, C0, 3, 3);
    conv("input_conv.conv2", C0, C0, 3, 3);
    for (size_t i = 0; i < cfg.blocks.size(); ++i) {
      const CodecBlockCfg& b = cfg.blocks[i];
      const std::string p = "decoder_blocks." + std::to_string(i);
      check_shape(w.tensor(p + ".conv_transpose.weight"), p + ".conv_transpose.weight",
                  {b.in_ch, b.out_ch, b.kth, b.ktw});
      check_shape(w.tensor(p + ".conv_transpose.bias"), p + ".conv_transpose.bias", {b.out_ch});
      conv(p + ".conv", b.out_ch, b.out_ch, b.kph, b.kpw);
      if (b.in_ch != b.out_ch) conv(p + ".shortcut", b.out_ch, b.in_ch, 1, 1);
    }
    conv("output_conv", cfg.out_ch, cfg.blocks.back().out_ch, cfg.out_k, cfg.out_k);
    const HostTensor& cb = cbs.tensor("codebooks");
    MRT_REQUIRE(cb.shape.size() == 3 && cb.shape[1] == cfg.codebook && cb.shape[2] == E &&
                    cb.shape[0] >= cfg.levels,
                "codec: codebooks must be (K >= levels, codebook, embedding_dim)");
  }
  MRT_HIP_CHECK(hipSetDevice(device));
  MRT_HIP_CHECK(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking));
  MRT_HIP_CHECK(hipEventCreate(&ev_[0]));
  MRT_HIP_CHECK(hipEventCreate(&ev_[1]));

  const HostTensor& cb = cbs.tensor("codebooks");
  const size_t cbn = static_cast<size_t>(cfg.levels) * cfg.codebook * E;
  codebooks_ = dalloc(cbn);
  MRT_HIP_CHECK(hipMemcpy(codebooks_, cb.data, cbn * 4, hipMemcpyHostToDevice));

  proj_c1_ = pack_conv(w, "input_proj.conv1", P, E, 1, 1);
  proj_c2_ = pack_conv(w, "input_proj.conv2", P, P, 1, 1);
  proj_sc_ = pack_conv(w, "input_proj.shortcut", P, E, 1, 1);
  in_c1_ = pack_conv(w, "input_conv.conv1", C0, C0, 3, 3);
  in_c2_ = pack_conv(w, "input_conv.conv2", C0, C0, 3, 3);
  for (size_t i = 0; i < cfg.blocks.size(); ++i) {
    const CodecBlockCfg& b = cfg.blocks[i];
    const std::string p = "decoder_blocks." + std::to_string(i);
    blk_t_.push_back(pack_transposed(w, p + ".conv_transpose", b.in_ch, b.out_ch, b.kth, b.ktw, b.sh, b.sw));
    blk_c_.push_back(pack_conv(w, p + ".conv", b.out_ch, b.out_ch, b.kph, b.kpw));
    blk_sc_.push_back(b.in_ch != b.out_ch ? pack_conv(w, p + ".shortcut", b.out_ch, b.in_ch, 1, 1) : Conv{});
  }
  {  // output conv: compact (kh, kw, cin, 2) for the vector-ALU kernel
    const int ci = cfg.blocks.back().out_ch, k = cfg.out_k;
    MRT_REQUIRE(k == 7 && ci % 8 == 0, "codec: output conv shape");
    const HostTensor& t = w.tensor("output_conv.weight");
    std::vector<float> h(static_cast<size_t>(k) * k * ci * 2);
    for (int o = 0; o < 2; ++o)
      for (int c = 0; c < ci; ++c)
        for (int y = 0; y < k; ++y)
          for (int x = 0; x < k; ++x)
            h[((static_cast<size_t>(y) * k + x) * ci + c) * 2 + o] = t.data[((static_cast<size_t>(o) * ci + c) * k + y) * k + x];
    out_w_ = dalloc(h.size());
    MRT_HIP_CHECK(hipMemcpy(out_w_, h.data(), h.size() * 4, hipMemcpyHostToDevice));
    out_b_ = dalloc(2);
    MRT_HIP_CHECK(hipMemcpy(out_b_, w.tensor("output_conv.bias").data, 8, hipMemcpyHostToDevice));
  }

  // iSTFT basis (spectrostream.cpp:616-646): frame row [re_0, im_0, .., re_479,
  // im_479] (bin 480, the restored Nyquist bin, is 0) -> windowed samples:
  // irfft = (re_0 + 2 sum_k (re_k cos - im_k sin)(2 pi k t / N)) / N, times the
  // synthesis window hann / (sum of hann^2 over the two hop phases).
  {
    const int N = cfg.n_fft, hop = cfg.hop, F = hop;
    std::vector<double> win(N), syn(N);
    for (int t = 0; t < N; ++t) win[t] = 0.5 - 0.5 * std::cos(2.0 * M_PI * t / N);
    for (int t = 0; t < N; ++t) {
      const double per = win[t % hop] * win[t % hop] + win[t % hop + hop] * win[t % hop + hop];
      syn[t] = win[t] / per;
    }
    istft_.cin = 2 * F;
    istft_.cout = N;
    istft_.cout_pad = round_up(N, 64);
    std::vector<float> h(static_cast<size_t>(2 * F) * istft_.cout_pad, 0.f);
    for (int k = 0; k < F; ++k)
      for (int t = 0; t < N; ++t) {
        const long kt = (static_cast<long>(k) * t) % N;
        const double ang = 2.0 * M_PI * static_cast<double>(kt) / N;
        const double c = k == 0 ? 1.0 : 2.0;
        h[static_cast<size_t>(2 * k) * istft_.cout_pad + t] = static_cast<float>(c * std::cos(ang) / N * syn[t]);
        h[static_cast<size_t>(2 * k + 1) * istft_.cout_pad + t] =
            static_cast<float>(-c * std::sin(ang) / N * syn[t]);
      }
    float* d = dalloc(h.size());
    MRT_HIP_CHECK(hipMemcpy(d, h.data(), h.size() * 4, hipMemcpyHostToDevice));
    istft_.w.push_back(d);
  }

  // activations at max_frames
  const int Hn = max_frames + cfg.temporal_pad;
  tok_ = static_cast<int*>(static_cast<void*>(dalloc(static_cast<size_t>(max_frames) * cfg.levels)));
  emb_ = dalloc(static_cast<size_t>(Hn) * E);
  skip_ = dalloc(static_cast<size_t>(Hn) * P);
  p1_ = dalloc(static_cast<size_t>(Hn) * P);
  x0_ = dalloc(static_cast<size_t>(Hn) * P);
  x0e_ = dalloc(static_cast<size_t>(Hn) * P);
  t0_ = dalloc(static_cast<size_t>(Hn) * P);
  x1_ = dalloc(static_cast<size_t>(Hn) * P);
  x1e_ = dalloc(static_cast<size_t>(Hn) * P);
  size_t tmax = 0, rmax = 0;
  int n = 1, H = Hn, W = cfg.unfold;
  for (size_t i = 0; i < cfg.blocks.size(); ++i) {
    const CodecBlockCfg& b = cfg.blocks[i];
    if (b.in_ch != b.out_ch) rmax = std::max(rmax, static_cast<size_t>(n) * H * W * b.out_ch);
    H *= b.sh;
    W *= b.sw;
    const size_t outn = static_cast<size_t>(n) * H * W * b.out_ch;
    tmax = std::max(tmax, outn);
    blk_out_.push_back(dalloc(outn));
    blk_oute_.push_back(dalloc(outn));
    blk_out_n_.push_back(outn);
    if (i == 0) n = 2;
  }
  MRT_REQUIRE(W == cfg.hop, "codec: the decoder's width must reach hop frequency bins");
  tbuf_ = dalloc(tmax);
  rbuf_ = dalloc(std::max<size_t>(rmax, 1));
  const int Hs = H - cfg.temporal_crop;
  spec_ = dalloc(static_cast<size_t>(2) * Hs * cfg.hop * 2);
  wf_ = dalloc(static_cast<size_t>(2) * Hs * cfg.n_fft);
  audio_ = dalloc(static_cast<size_t>(max_frames) * cfg.samples_per_frame * 2);
}

Codec::~Codec() {
  (void)hipSetDevice(device);
  if (stream) (void)hipStreamSynchronize(stream);
  for (auto& kv : plans_)
    if (kv.second->subs_dev) (void)hipFree(kv.second->subs_dev);
  for (void* p : allocs_) (void)hipFree(p);
  for (hipEvent_t e : ev_)
    if (e) (void)hipEventDestroy(e);
  if (stream) (void)hipStreamDestroy(stream);
}

// The launches of one decode of `frames` frames.  Every sub-problem's output
// and residual coordinates are checked against their buffers here, on the
// host, before anything is launched (input coordinates are bounds-checked in
// the kernel, where out-of-range taps read the zero padding).
const Codec::Plan& Codec::plan(int frames) {
  auto it = plans_.find(frames);
  if (it != plans_.end()) return *it->second;
  auto pl = std::make_unique<Plan>();
  pl->frames = frames;
  std::vector<std::vector<ConvSub>> subs;
  size_t need_partial = 0;

  auto add = [&](ConvLaunch L, std::vector<ConvSub> s) {
    int tiles = 0;
    for (auto& q : s) {
      q.tile0 = tiles;
      const long M = static_cast<long>(L.n) * q.gy * q.gx;
      MRT_REQUIRE(M >= 1 && q.ntaps >= 1 && q.ntaps <= kConvMaxTaps, "codec plan: empty sub-problem");
      tiles += static_cast<int>((M + 63) / 64);
      // output / residual coordinates at the grid's corners (affine, monotone)
      for (int y : {0, q.gy - 1})
        for (int x : {0, q.gx - 1}) {
          const int oy = y * q.oys + q.oyo, ox = x * q.oxs + q.oxo;
          MRT_REQUIRE(oy >= 0 && oy < L.hout && ox >= 0 && ox < L.wout, "codec plan: output out of range");
          if (L.res)
            MRT_REQUIRE(oy / L.rh < L.res_h && ox / L.rw < L.res_w, "codec plan: residual out of range");
        }
    }
    MRT_REQUIRE(L.cin % 16 == 0 && L.cout % L.split == 0, "codec plan: channel layout");
    // split-K when the tiles alone give fewer than 2 workgroups per CU:
    // ~512 workgroups, >= 2 K chunks per slice
    L.ksplit = 1;
    L.rows = tiles * 64;
    const int blocks = tiles * (L.cout_pad / 64);
    if (blocks < 512) {
      int min_nk = 1 << 30;
      for (auto& q : s) min_nk = std::min(min_nk, q.ntaps * (L.cin / (L.cin % 32 == 0 ? 32 : 16)));
      L.ksplit = std::max(1, std::min({(512 + blocks - 1) / blocks, min_nk / 2, 16}));
    }
    if (L.ksplit > 1) need_partial = std::max(need_partial, static_cast<size_t>(L.ksplit) * L.rows * L.cout_pad);
    pl->launches.push_back(L);
    pl->tiles_m.push_back(tiles);
    pl->tiles_n.push_back(L.cout_pad / 64);
    subs.push_back(std::move(s));
  };
  auto base = [&](const Conv& c, const float* x, int n, int hin, int win, float* y, int hout, int wout) {
    ConvLaunch L{};
    L.x = x;
    L.n = n;
    L.hin = hin;
    L.win = win;
    L.cin = c.cin;
    L.y = y;
    L.hout = hout;
    L.wout = wout;
    L.cout = c.cout;
    L.split = c.cout;
    L.cout_pad = c.cout_pad;
    L.bias = c.bias;
    L.rh = L.rw = 1;
    return L;
  };
  // a stride-1 convolution with taps (kh, kw) reading (y + kh - top + shift, x + kw - left)
  auto regular = [&](const Conv& c, int H, int W, int kh, int kw, int top, int left, int shift) {
    ConvSub s{};
    s.gy = H;
    s.gx = W;
    s.oys = s.oxs = 1;
    s.ntaps = kh * kw;
    s.w = c.w[0];
    for (int y = 0; y < kh; ++y)
      for (int x = 0; x < kw; ++x) {
        s.dy[y * kw + x] = static_cast<int16_t>(y - top + shift);
        s.dx[y * kw + x] = static_cast<int16_t>(x - left);
      }
    return std::vector<ConvSub>{s};
  };

  const int Hn = frames + cfg.temporal_pad;
  // Res1x1Block input_proj (spectrostream.cpp:174-181) on (1, Hn, 1, E)
  add(base(proj_sc_, emb_, 1, Hn, 1, skip_, Hn, 1), regular(proj_sc_, Hn, 1, 1, 1, 0, 0, 0));
  {
    ConvLaunch L = base(proj_c1_, emb_, 1, Hn, 1, p1_, Hn, 1);
    L.act_out = kActElu;
    add(L, regular(proj_c1_, Hn, 1, 1, 1, 0, 0, 0));
    ConvLaunch L2 = base(proj_c2_, p1_, 1, Hn, 1, x0_, Hn, 1);
    L2.y_elu = x0e_;  // elu(x0): input_conv's first conv reads it as is
    L2.res = skip_;
    L2.res_h = Hn;
    L2.res_w = 1;
    add(L2, regular(proj_c2_, Hn, 1, 1, 1, 0, 0, 0));
  }
  // unfold_width(5) is a reshape: (1, Hn, 1, P) == (1, Hn, 5, C0).
  const int W0 = cfg.unfold;
  // Res3x3Block input_conv, causal (spectrostream.cpp:191-200): pads top 2, left 1
  {
    ConvLaunch L = base(in_c1_, x0e_, 1, Hn, W0, t0_, Hn, W0);
    L.act_out = kActElu;
    add(L, regular(in_c1_, Hn, W0, 3, 3, 2, 1, 0));
    ConvLaunch L2 = base(in_c2_, t0_, 1, Hn, W0, x1_, Hn, W0);
    L2.y_elu = x1e_;
    L2.res = x0_;
    L2.res_h = Hn;
    L2.res_w = W0;
    add(L2, regular(in_c2_, Hn, W0, 3, 3, 2, 1, 0));
  }
  // DecoderResBlocks (spectrostream.cpp:224-262)
  const float* x = x1_;   // raw: the residual / shortcut input
  const float* xe = x1e_;  // elu(x): the transposed conv's input
  int n = 1, H = Hn, W = W0;
  for (size_t i = 0; i < cfg.blocks.size(); ++i) {
    const CodecBlockCfg& b = cfg.blocks[i];
    const int Ho = H * b.sh, Wo = W * b.sw;  // (H - 1) s + k minus the crop k - s
    const int cs = (b.ktw - b.sw) / 2;       // crop_w_start
    const float* res = x;
    if (b.in_ch != b.out_ch) {  // shortcut on the input grid, repeated by the epilogue below
      add(base(blk_sc_[i], x, n, H, W, rbuf_, H, W), regular(blk_sc_[i], H, W, 1, 1, 0, 0, 0));
      res = rbuf_;
    }
    // conv_transpose(elu(x)) + bias, cropped, then elu: one sub-problem per phase
    {
      ConvLaunch L = base(blk_t_[i], xe, n, H, W, tbuf_, Ho, Wo);
      L.act_out = kActElu;
      std::vector<ConvSub> ph_subs;
      int wi = 0;
      for (int ph = 0; ph < b.sh; ++ph)
        for (int pw = 0; pw < b.sw; ++pw) {
          const int nj = (b.kth - ph + b.sh - 1) / b.sh, ni = (b.ktw - pw + b.sw - 1) / b.sw;
          const int qx0 = cs > pw ? (cs - pw + b.sw - 1) / b.sw : 0;
          ConvSub s{};
          s.oys = b.sh;
          s.oyo = ph;
          s.oxs = b.sw;
          s.oxo = qx0 * b.sw + pw - cs;
          s.gy = (Ho - ph + b.sh - 1) / b.sh;
          s.gx = (Wo - s.oxo + b.sw - 1) / b.sw;
          s.ntaps = nj * ni;
          s.w = blk_t_[i].w[wi++];
          for (int j = 0; j < nj; ++j)
            for (int q = 0; q < ni; ++q) {
              s.dy[j * ni + q] = static_cast<int16_t>(-j);
              s.dx[j * ni + q] = static_cast<int16_t>(qx0 - q);
            }
          if (s.gy >= 1 && s.gx >= 1) ph_subs.push_back(s);
        }
      add(L, std::move(ph_subs));
    }
    // conv(causal pad(elu'd T)) + bias + residual (repeated by the stride)
    {
      const int top = b.kph - 1, left = (b.kpw - 1) / 2;
      ConvLaunch L = base(blk_c_[i], tbuf_, n, Ho, Wo, blk_out_[i], Ho, Wo);
      L.y_elu = blk_oute_[i];
      L.res = res;
      L.res_h = H;
      L.res_w = W;
      L.rh = b.sh;
      L.rw = b.sw;
      if (i == 0) L.split = b.out_ch / 2;  // stereo split (spectrostream.cpp:384-392)
      add(L, regular(blk_c_[i], Ho, Wo, b.kph, b.kpw, top, left, 0));
    }
    x = blk_out_[i];
    xe = blk_oute_[i];
    if (i == 0) n = 2;
    H = Ho;
    W = Wo;
  }
  // elu -> output conv 7x7 causal, first temporal_crop rows dropped (out_conv)
  const int Hs = H - cfg.temporal_crop;
  MRT_REQUIRE(x == blk_out_.back() && Hs >= 1, "codec plan: output conv input");
  pl->out_at = static_cast<int>(pl->launches.size());
  pl->out_h = H;
  pl->out_w = W;
  pl->out_hs = Hs;
  // iSTFT frames: spec (2 Hs rows of 2 hop) x basis (2 hop, n_fft)
  add(base(istft_, spec_, 1, 2 * Hs, 1, wf_, 2 * Hs, 1), regular(istft_, 2 * Hs, 1, 1, 1, 0, 0, 0));

  if (need_partial > partial_n_) {
    MRT_HIP_CHECK(hipStreamSynchronize(stream));  // an older, smaller buffer may still be in use
    partial_ = dalloc(need_partial);
    partial_n_ = need_partial;
  }
  for (auto& L : pl->launches) L.partial = partial_;
  // upload every launch's sub-problems into one device array
  size_t total = 0;
  for (auto& s : subs) total += s.size();
  MRT_HIP_CHECK(hipMalloc(&pl->subs_dev, total * sizeof(ConvSub)));
  std::vector<ConvSub> flat;
  flat.reserve(total);
  for (size_t l = 0; l < subs.size(); ++l) {
    pl->launches[l].subs = pl->subs_dev + flat.size();
    pl->launches[l].nsub = static_cast<int>(subs[l].size());
    flat.insert(flat.end(), subs[l].begin(), subs[l].end());
  }
  MRT_HIP_CHECK(hipMemcpy(pl->subs_dev, flat.data(), total * sizeof(ConvSub), hipMemcpyHostToDevice));
  Plan& ref = *pl;
  plans_[frames] = std::move(pl);
  return ref;
}

void Codec::enqueue(const int* tokens_dev, int frames, float* audio_dev) {
  const Plan& pl = plan(frames);
  MRT_HIP_CHECK(hipEventRecord(ev_[0], stream));
  rvq_dequant(tokens_dev, frames, cfg.levels, codebooks_, cfg.codebook, cfg.embedding_dim, cfg.temporal_pad, emb_,
              stream);
  for (size_t l = 0; l < pl.launches.size(); ++l) {
    if (static_cast<int>(l) == pl.out_at)
      out_conv(blk_oute_.back(), 2, pl.out_h, pl.out_w, cfg.blocks.back().out_ch, cfg.temporal_crop, false, out_w_,
               out_b_,
               spec_, pl.out_hs, stream);
    conv_launch(pl.launches[l], pl.tiles_m[l], pl.tiles_n[l], stream);
  }
  const int Hs = spec_frames(frames);
  overlap_add(wf_, Hs, cfg.n_fft, frames * cfg.samples_per_frame, audio_dev, stream);
  MRT_HIP_CHECK(hipEventRecord(ev_[1], stream));
  timed_ = true;
  last_frames_ = frames;
}

void Codec::decode(const int32_t* tokens_host, int frames, float* audio_host) {
  MRT_REQUIRE(tokens_host && audio_host, "codec: null buffer");
  MRT_REQUIRE(frames >= 1 && frames <= max_frames, "codec: frames must be in [1, max_frames]");
  const size_t nt = static_cast<size_t>(frames) * cfg.levels;
  for (size_t i = 0; i < nt; ++i)
    MRT_REQUIRE(tokens_host[i] >= 0 && tokens_host[i] < cfg.codebook,
                "rvq_dequantization: token id outside [0, codebook_size)");
  MRT_HIP_CHECK(hipSetDevice(device));
  MRT_HIP_CHECK(hipMemcpyAsync(tok_, tokens_host, nt * 4, hipMemcpyHostToDevice, stream));
  enqueue(tok_, frames, audio_);
  const size_t na = static_cast<size_t>(frames) * cfg.samples_per_frame * 2;
  MRT_HIP_CHECK(hipMemcpyAsync(audio_host, audio_, na * 4, hipMemcpyDeviceToHost, stream));
  MRT_HIP_CHECK(hipStreamSynchronize(stream));
}

void Codec::decode_device(const int* tokens_dev, int frames, float* audio_dev) {
  MRT_REQUIRE(tokens_dev && audio_dev, "codec: null buffer");
  MRT_REQUIRE(frames >= 1 && frames <= max_frames, "codec: frames must be in [1, max_frames]");
  MRT_HIP_CHECK(hipSetDevice(device));
  enqueue(tokens_dev, frames, audio_dev);
}

float Codec::last_ms() const {
  if (!timed_) return 0.f;
  MRT_HIP_CHECK(hipEventSynchronize(ev_[1]));
  float ms = 0.f;
  MRT_HIP_CHECK(hipEventElapsedTime(&ms, ev_[0], ev_[1]));
  return ms;
}

std::pair<const void*, size_t> Codec::buffer(int which) const {
  const int f = last_frames_ > 0 ? last_frames_ : max_frames;
  const int Hn = f + cfg.temporal_pad;
  const size_t fl = 4;
  if (which == kCodecEmb) return {emb_, fl * Hn * cfg.embedding_dim};
  if (which == kCodecInputConv) return {x1_, fl * Hn * cfg.proj_ch};
  if (which >= kCodecBlock0 && which < kCodecBlock0 + static_cast<int>(cfg.blocks.size())) {
    const int i = which - kCodecBlock0;
    // block i output at f frames: blocks' spatial sizes scale with Hn
    int n = 1, H = Hn, W = cfg.unfold;
    size_t cnt = 0;
    for (int k = 0; k <= i; ++k) {
      H *= cfg.blocks[k].sh;
      W *= cfg.blocks[k].sw;
      cnt = static_cast<size_t>(n) * H * W * cfg.blocks[k].out_ch;
      if (k == 0) n = 2;
    }
    return {blk_out_[i], fl * cnt};
  }
  if (which == kCodecSpec) return {spec_, fl * 2 * spec_frames(f) * cfg.hop * 2};
  if (which == kCodecFrames) return {wf_, fl * 2 * spec_frames(f) * cfg.n_fft};
  throw Error(1, "codec: unknown buffer id");
}

}  // namespace mrt
