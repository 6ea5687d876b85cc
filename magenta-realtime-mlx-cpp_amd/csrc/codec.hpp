// Codec decode on the device: RVQ dequantisation (rvq.cpp:68-88), the
// SpectroStream decoder (spectrostream.cpp:163-432) and the iSTFT
// post-processor (spectrostream.cpp:593-681), in fp32 as the reference runs
// it (system.cpp:118-119, 373-390).
//
// Every convolution is an implicit GEMM on the fp32 matrix cores
// (codec_kernels.hip): M = output pixels, N = output channels, K = taps x
// input channels, activations NHWC.  A transposed convolution is launched as
// one sub-problem per output stride phase, each a stride-1 convolution over
// the input (no multiplies by inserted zeros); crops are output offsets; the
// ELUs, biases and residual adds are fused into the operand loads and the
// epilogue; a block's 1x1 shortcut runs on its input grid (it commutes with
// the residual's repeat).  The iSTFT is one GEMM against a windowed real-DFT
// basis followed by an overlap-add kernel.
#pragma once

#include <cstdint>
#include <map>
#include <memory>
#include <vector>

#include "common.hpp"
#include "safetensors.hpp"

namespace mrt {

constexpr int kConvMaxTaps = 49;
// Epilogue activations: ELU (nn_ops.h:31-39), exact GELU x/2 (1 + erf(x/sqrt 2)) (nn_ops.h:41-53).
constexpr int kActNone = 0, kActElu = 1, kActGelu = 2;

// One stride-1 sub-problem of a convolution launch.  GEMM row m = (n, y, x)
// over an n x gy x gx grid; output pixel (y * oys + oyo, x * oxs + oxo); tap t
// reads input pixel (y + dy[t], x + dx[t]) (zero outside the input) against
// packed weights w[(t * cin + c) * cout_pad + o].
struct ConvSub {
  int gy, gx;
  int oys, oyo, oxs, oxo;
  int ntaps;
  int tile0;  // first M tile of this sub-problem in the launch
  const float* w;
  int16_t dy[kConvMaxTaps];
  int16_t dx[kConvMaxTaps];
};

struct ConvLaunch {
  const float* x;  // (n, hin, win, cin)
  int n, hin, win, cin;
  float* y;  // (n * cout / split, hout, wout, split): output channel o of image b goes to
             // image (o / split) * n + b, channel o % split
  int hout, wout, cout, split, cout_pad;
  const float* bias;  // (cout)
  const float* res;   // (n, res_h, res_w, cout) added at (oy / rh, ox / rw), or null
  int res_h, res_w, rh, rw;
  int elu_in;   // ELU on the loaded input (zero padding stays 0)
  int act_out;  // on the result: kActNone, kActElu or kActGelu
  int nsub;
  const ConvSub* subs;  // device array of nsub
  // split-K: ksplit > 1 splits each tile's K loop over blockIdx.z; the slices
  // write raw sums to partial[(z * rows + tile row) * cout_pad + o] (rows =
  // 64 x the launch's M tiles) and conv_finish adds them in slice order
  // before the epilogue.
  int ksplit, rows;
  float* partial;
  float* y_elu;  // when non-null, also elu(result) here (same layout): the next ELU'd input
};

// One convolution launch (plus its split-K finish when a.ksplit > 1).
void conv_launch(const ConvLaunch& a, int tiles_m, int tiles_n, hipStream_t s);
// emb (frames + pad, dim): rows < frames = sum over levels k < levels of
// codebooks[k][tokens[f * levels + k]] (fp32, level order); the pad rows 0.
// Ids outside [0, codebook) are read as 0.
void rvq_dequant(const int* tokens, int frames, int levels, const float* codebooks, int codebook, int dim, int pad,
                 float* emb, hipStream_t s);
// The output conv: x (n, H, W, cin) -> out (n, Hs, W, 2) = conv7x7(elu(x))
// (x already ELU'd when !elu_in) with causal padding (top 6, left 3, right 3)
// over input rows from `crop` on, plus bias; w packed (kh, kw, cin, 2); cin a
// multiple of 8.
void out_conv(const float* x, int n, int H, int W, int cin, int crop, bool elu_in, const float* w, const float* bias,
              float* out, int Hs, hipStream_t s);
// audio (T, 2) from windowed frames wf (2 * H, n_fft): overlap-add at hop
// n_fft / 2 (spectrostream.cpp:649-667), trimmed to T, channels interleaved.
void overlap_add(const float* wf, int H, int n_fft, int T, float* audio, hipStream_t s);

struct CodecBlockCfg {
  int in_ch, out_ch, sh, sw, kth, ktw, kph, kpw;
};

struct CodecConfig {
  int embedding_dim = 256, proj_ch = 2560, unfold = 5;
  std::vector<CodecBlockCfg> blocks = {
      {512, 1024, 2, 1, 4, 3, 3, 3}, {512, 256, 2, 2, 4, 4, 3, 3}, {256, 256, 1, 2, 3, 4, 3, 3},
      {256, 256, 1, 2, 3, 4, 3, 3},  {256, 128, 1, 3, 3, 6, 3, 3}, {128, 128, 1, 2, 3, 4, 3, 3},
      {128, 64, 1, 2, 3, 4, 3, 3}};
  int out_ch = 2, out_k = 7;
  int temporal_pad = 1, temporal_crop = 4;
  int n_fft = 960, hop = 480, samples_per_frame = 1920;
  int levels = 16, codebook = 1024;
};

// Buffer ids for Codec::buffer (parity / inspection).
enum CodecBuf : int {
  kCodecEmb = 0,        // (frames + 1, E)
  kCodecInputConv = 1,  // (1, frames + 1, unfold, proj / unfold)
  kCodecBlock0 = 2,     // .. kCodecBlock0 + 6: block outputs (stereo-split after block 0)
  kCodecSpec = 9,       // (2, H, 480, 2) planar: image s, channel (real, imag)
  kCodecFrames = 10,    // (2 H, n_fft) windowed iSTFT frames
};

class Codec {
 public:
  // w: decoder bundle; cb: the bundle holding "codebooks" (may be the same source).
  Codec(const TensorSource& w, const TensorSource& cb, const CodecConfig& c, int device, int max_frames);
  ~Codec();
  Codec(const Codec&) = delete;
  Codec& operator=(const Codec&) = delete;

  const CodecConfig cfg;
  const int device, max_frames;
  hipStream_t stream = nullptr;

  // tokens: host (frames, levels) RVQ ids; audio: host (frames * 1920, 2).
  void decode(const int32_t* tokens_host, int frames, float* audio_host);
  // Device pointers; enqueued on `stream`, no host sync.
  void decode_device(const int* tokens_dev, int frames, float* audio_dev);
  // Builds (and checks) the launch plan of a decode of `frames` frames now,
  // so that a later decode of that size cannot fail on its geometry.
  void prepare(int frames) {
    MRT_REQUIRE(frames >= 1 && frames <= max_frames, "codec: frames must be in [1, max_frames]");
    MRT_HIP_CHECK(hipSetDevice(device));
    plan(frames);
  }
  float last_ms() const;
  // (pointer, bytes) of an intermediate of the last decode.
  std::pair<const void*, size_t> buffer(int which) const;
  int spec_frames(int frames) const { return 4 * (frames + cfg.temporal_pad) - cfg.temporal_crop; }

 private:
  struct Conv {  // packed GEMM weights of one convolution (one entry per sub-problem)
    std::vector<float*> w;
    float* bias = nullptr;
    int cin = 0, cout = 0, cout_pad = 0;
  };
  struct Plan {
    std::vector<ConvLaunch> launches;
    std::vector<int> tiles_m, tiles_n;
    ConvSub* subs_dev = nullptr;
    int frames = 0;
    int out_at = 0;  // the output conv runs before launches[out_at]
    int out_h = 0, out_w = 0, out_hs = 0;
  };
  const Plan& plan(int frames);
  void enqueue(const int* tokens_dev, int frames, float* audio_dev);
  float* dalloc(size_t floats);
  Conv pack_conv(const TensorSource& w, const std::string& name, int o, int i, int kh, int kw);
  Conv pack_transposed(const TensorSource& w, const std::string& name, int i, int o, int kh, int kw, int sh, int sw);

  std::vector<void*> allocs_;
  float* codebooks_ = nullptr;
  Conv proj_sc_, proj_c1_, proj_c2_, in_c1_, in_c2_, istft_;
  float *out_w_ = nullptr, *out_b_ = nullptr;  // output conv (kh, kw, cin, 2), bias (2)
  std::vector<Conv> blk_t_, blk_c_, blk_sc_;
  float *emb_ = nullptr, *skip_ = nullptr, *p1_ = nullptr, *x0_ = nullptr, *t0_ = nullptr, *x1_ = nullptr;
  float *x0e_ = nullptr, *x1e_ = nullptr;  // elu(x0), elu(x1)
  std::vector<float*> blk_out_, blk_oute_;  // block outputs and their ELU'd copies
  std::vector<size_t> blk_out_n_;
  float *tbuf_ = nullptr, *rbuf_ = nullptr, *spec_ = nullptr, *wf_ = nullptr, *audio_ = nullptr;
  int* tok_ = nullptr;
  int last_frames_ = 0;
  std::map<int, std::unique_ptr<Plan>> plans_;
  float* partial_ = nullptr;  // split-K partial sums (grown by plan())
  size_t partial_n_ = 0;
  hipEvent_t ev_[2] = {nullptr, nullptr};
  bool timed_ = false;
};

}  // namespace mrt
