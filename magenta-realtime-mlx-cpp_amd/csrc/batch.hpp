// Batched independent streams: B streams (each its own encoder tokens, seed,
// KV caches) decoded together as R = 2B activation rows, so every projection
// is one skinny GEMM on the matrix cores and the weights stream once per step
// for all streams.  Per stream the semantics are those of generate_tokens
// (depthformer/decode.cpp:239-573) at batch 1.
#pragma once

#include <cstdint>
#include <vector>

#include "common.hpp"
#include "model.hpp"

namespace mrt {

constexpr int kBatchRows = 64;  // activation rows of one batched step (32 streams)

// RMSNorm (eps, weights g) of a GEMM's input rows applied as they are loaded:
// X then holds the raw residual rows, whose sums of squares are the K / 16
// partials per row (row-major, K / 16 a row) that the bgemm_resid which last
// wrote them left at ssq.  g == nullptr: X is used as it is.
struct BNorm {
  const void* g = nullptr;
  const float* ssq = nullptr;
  float eps = 0.f;
};

// Skinny GEMMs Y (M x N) = X (M x K) . W^T, bf16 in, fp32 accumulation, M <= 64,
// K % 32 == 0 (batch_kernels.hip).  Epilogues as the batch-1 GEMVs.
void bgemm_store(const void* X, int M, int K, const void* W, int N, void* Y, int ldy, hipStream_t s,
                 const BNorm& norm = {});
void bgemm_f32(const void* X, int M, int K, const void* W, int N, float* Y, int ldy, hipStream_t s,
               const BNorm& norm = {});
// R += X . W^T (rounded as the batch-1 residual); ssq non-null: each updated
// row's sums of squares over its 16-column tiles, (M, N / 16) floats.
void bgemm_resid(const void* X, int M, int K, const void* W, int N, void* R, int ldr, hipStream_t s,
                 float* ssq = nullptr);
// W = [Wq; Wk; Wv] (3 HD rows): q -> Q (M, HD); k, v -> ring slot pos (or
// *pos_ptr when non-null) of caches laid out (M, H, Lmax, 64).
void bgemm_qkv(const void* X, int M, int K, const void* W, int HD, void* Q, void* Kc, void* Vc, int H, int Lmax, int pos,
               const int* pos_ptr, hipStream_t s, const BNorm& norm = {});
// The same for rows m = P * pos + r (positions of one stream's frame, P CFG
// rows each): k / v -> slot pos of ring row r (P, H, Lmax, 64).
void bgemm_qkv_pos(const void* X, int M, int K, const void* W, int HD, void* Q, void* Kc, void* Vc, int H, int Lmax,
                   int P, hipStream_t s);
// groups independent products: rows [g rows, +rows) of X against
// W + g * w_group_stride, logits rounded to bf16 into Y rows g rows + m.
void bgemm_f32_grouped(const void* X, int rows, int K, const void* W, long w_group_stride, int N, float* Y, int ldy,
                       int groups, hipStream_t s);
// Gated GELU over the 32-row packed wi_0 / wi_1 matrix (2F rows) -> (M, F).
void bgemm_geglu(const void* X, int M, int K, const void* W01, int F, void* Hout, int ldh, hipStream_t s,
                 const BNorm& norm = {});

// Cross attention (no bias, no mask, scale 1) of every (row, head) over S <=
// 1024 encoder keys, caches laid out (rows, H, S, 64); out (rows, H * 64).
void cross_attn_rows(const void* Q, const void* Kc, const void* Vc, int rows, int H, int S, void* out, hipStream_t s);

// Gumbel noise of every draw for every stream: out (streams, frames, L, C).
void gumbel_tables(const uint64_t* seeds, int streams, int frames, int L, int C, float* out, hipStream_t s);

// Device frame counter of a replayed frame graph.
void set_counter(int* p, int v, hipStream_t s);
void advance_counter(int* p, hipStream_t s);

class Batch {
 public:
  Batch(Model& m, int streams, int max_frames, int enc_len);
  ~Batch();
  Batch(const Batch&) = delete;
  Batch& operator=(const Batch&) = delete;

  Model& m;
  int B, R, F, S;
  hipStream_t stream = nullptr;

  // tokens: host (R, S); rows 2b and 2b + 1 are stream b's CFG pair.
  void encode(const int32_t* tokens_host);
  void encode_device();
  int* enc_tokens_dev() const { return enc_.tok; }
  // One chunk of every stream.  seeds: host (B); o.teacher: host (B, F, L)
  // or null; out: host (B, num_frames, L) LLM ids.  o.record_slices (device
  // (F, L, R, C)) and o.record_temporal (device (F, R, D)) run the loop
  // without the frame graph.
  void generate(const int32_t* enc_tokens_host, const GenOpts& o, const uint64_t* seeds, int32_t* out_host);
  // GPU ms of the last generate call's decode section.
  float last_decode_ms() const;
  void* enc_out() const { return enc_.enc_out; }

 private:
  void enqueue_frame(const GenOpts& o, int f, bool dynamic);
  void temporal_stack(int f, const int* fptr);
  void depth_stack(void* x, int l, bool x_partials, bool qkv_fed = false);
  // the norm (weights g) of a GEMM input whose row partials are at ssq_
  BNorm norm(const void* g) const { return BNorm{g, ssq_, 1e-6f}; }
  void* dalloc(size_t bytes);
  char* ring(void* base, int layer, int kv, int len) const;

  std::vector<void*> allocs_;
  EncoderBufs enc_;
  bool encoded_ = false;
  void *tkv_ = nullptr, *dkv_ = nullptr;
  void *t_in_ = nullptr, *d_in_ = nullptr, *xn_ = nullptr, *q_ = nullptr, *att_ = nullptr, *ffh_ = nullptr;
  float* ssq_ = nullptr;  // row partials of the last residual update: (R, d_model / 16)
  // the model's depth layer-0 q/k/v table of the current call's codec levels,
  // or nullptr (layer 0 computed at every level)
  const void* qkv_tab_ = nullptr;
  void* fsum_ = nullptr;
  float* logits_ = nullptr;
  float* noise_ = nullptr;  // (B, F, L, 1024) Gumbel noise of the current call
  int *d_tokens_ = nullptr, *d_teacher_ = nullptr, *d_frame_ = nullptr;
  uint64_t* d_seeds_ = nullptr;
  int32_t* h_pinned_ = nullptr;
  size_t h_pinned_n_ = 0;
  hipEvent_t ev_[2] = {nullptr, nullptr};
  bool timed_ = false;
  hipGraph_t graph_ = nullptr;
  hipGraphExec_t graph_exec_ = nullptr;
  std::vector<double> graph_key_;
};

}  // namespace mrt
