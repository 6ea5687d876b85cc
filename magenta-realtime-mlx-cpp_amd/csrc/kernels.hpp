// Host-side launchers for the Depthformer HIP kernels (gfx950).
//
// Conventions shared by every launcher:
//   * ``T`` is the model storage type selected by ``DType`` (fp32, bf16 or fp16);
//     all accumulation is fp32.
//   * Linear weights are (out, in) row-major, exactly as the bundle stores
//     them (modules.h:74-76), so a GEMV row is one contiguous dot product.
//   * ``nb`` is the number of activation rows (2 = one CFG stream).
//   * Values the reference materialises in the model dtype are rounded to it
//     at the same points (identity for fp32).
#pragma once

#include "common.hpp"

namespace mrt {

// RMSNorm prologue applied to X before a GEMV/GEMM when ``g`` is non-null:
// x_hat = round(round(x * rsqrt(mean(x^2) + eps)) * g)   (modules.cpp:72-84).
struct NormArg {
  const void* g = nullptr;
  float eps = 1e-6f;
};

// ---- decode GEMVs: Y[b, n] = sum_k W[n, k] * X[b, k] ------------------------
// Plain store to Y (model dtype).
void gemv_store(DType dt, int nb, const void* W, int N, int K, const void* X, int ldx,
                NormArg norm, void* Y, int ldy, hipStream_t s);
// Store rounded-to-model-dtype values as fp32 (logits).
void gemv_f32(DType dt, int nb, const void* W, int N, int K, const void* X, int ldx,
              NormArg norm, float* Y, int ldy, hipStream_t s);
// Residual: R[b, n] = round(R[b, n] + round(Y[b, n])).
void gemv_resid(DType dt, int nb, const void* W, int N, int K, const void* X, int ldx,
                NormArg norm, void* R, int ldr, hipStream_t s);
// Fused q/k/v projection (W = [Wq; Wk; Wv], 3*HD rows). q goes to Q (nb, HD);
// k and v are written into ring slot ``pos`` of the caches laid out
// (nb, H, Lmax, 64).
void gemv_qkv(DType dt, int nb, const void* W, int HD, int K, const void* X, int ldx,
              NormArg norm, void* Q, void* Kc, void* Vc, int H, int Lmax, int pos,
              hipStream_t s);
// Gated-GELU: W01 packs wi_0/wi_1 in 32-row groups [gate 32 | up 32]; writes
// H[b, j] = round(gelu(round(gate)) * round(up)) for j < F.
void gemv_geglu(DType dt, int nb, const void* W01, int F, int K, const void* X, int ldx,
                NormArg norm, void* Hout, int ldh, hipStream_t s);

// ---- decode attention -------------------------------------------------------
// Self-attention of the query at ring position qpos over slots 0..len-1,
// scale 1.0, additive bias table[bucket[qpos - j], h] (modules.cpp:243-295).
// bias_row: an explicit bias (H, len) model dtype replacing the table lookup.
void self_attn(DType dt, int nb, const void* Q, const void* Kc, const void* Vc, int H,
               int Lmax, int len, int qpos, const void* bias_tab, const int* buckets,
               void* out, hipStream_t s, const void* bias_row = nullptr);
// The same with the query position read on the device from *qpos_ptr when it
// is non-null (len = qpos + 1; the caller keeps it below Lmax).
// pos_rows > 0 instead attends all positions of one frame at once: query row
// b is position b / pos_rows of ring row b % pos_rows, causal (len = pos + 1).
void self_attn_at(DType dt, int nb, const void* Q, const void* Kc, const void* Vc, int H, int Lmax, int len,
                  int qpos, const int* qpos_ptr, const void* bias_tab, const int* buckets, void* out,
                  hipStream_t s, int pos_rows = 0, const void* bias_row = nullptr);
// The rel-pos bias of steps 0..n-1 (precompute_{temporal,depth}_biases,
// model.cpp:302-320) back to back: step f's (H, f + 1) block at element
// H * f * (f + 1) / 2, entry [h][j] = table[bucket(f - j), h].
void bias_rows(DType dt, const void* table, const int* buckets, int H, int n, void* out, hipStream_t s);
// Self-attention of all K positions of nb sequences at once (the full-sequence
// depth pass): qkv (nb*K, 3*HD) rows m = b*K + i, [q | k | v]; query (b, i)
// attends keys (b, j) for j <= i (causal) or all j < K, with the bias
// explicit[(h*K + i)*K + j] when `explicit_bias` is set, else
// bias_tab[buckets[max(i - j, 0)] * H + h]; scale 1.0; out (nb*K, HD).  K <= 64.
void full_attn(DType dt, int nb, int K, int H, const void* qkv, const void* explicit_bias, const void* bias_tab,
               const int* buckets, bool causal, void* out, hipStream_t s);
// Cross-attention over S encoder keys (no bias/mask), split over key blocks.
// ``part`` needs nb*H*nsplit*66 floats.
void cross_attn(DType dt, int nb, const void* Q, const void* Kc, const void* Vc, int H,
                int S, void* out, float* part, int nsplit, hipStream_t s);
int cross_attn_splits(int S);

// out[r, :] = emb[ids[r], :] for r < rows (model dtype copy).
void embed_rows(DType dt, const void* emb, int D, const int* ids, int rows, void* out,
                hipStream_t s);
// out[r, :] = emb[id, :] for every r < rows.
void embed_fill(DType dt, const void* emb, int D, int id, int rows, void* out, hipStream_t s);
// Device-to-device copy as a kernel (kept out of memcpy graph nodes).
void copy_dev(void* dst, const void* src, size_t bytes, hipStream_t s);

// ---- sampling -----------------------------------------------------------------
struct SampleParams {
  float guidance_weight;
  float temperature;
  int top_k;
  int codebook;       // C: entries per level
  int codec_offset;   // first id of level 0
  int rvq_depth;      // L
  const uint64_t* seed;  // device pointer to the draw seed (one per stream), or nullptr: seed_value
  // Optional tabulated noise: noise[((stream * noise_frames + frame) * rvq_depth
  // + level) * codebook + i] = gumbel(seed[stream], frame, level, i).
  const float* noise = nullptr;
  int noise_frames = 0;
  // Optional: levels <= *decided already have their token (speculative
  // decoding); the sampler then only feeds emb(token) to next_in (no draw, no
  // frame sum) and the depth step returns at once.
  const int* decided = nullptr;
  // The draw seed of stream 0 when `seed` is nullptr (passed by value, so
  // calls that share no device buffer cannot see each other's seeds).
  uint64_t seed_value = 0;
};

// One CFG stream: rows (0, 1) of ``logits`` (nb=2, C) level slice.
// CFG-combine -> (temperature, top-k, Gumbel-max) or argmax -> token; the
// noise of candidate i is keyed by (seed, frame, level, i).
// Writes tokens[slot] (fed-back id: teacher[slot] if ``teacher`` is non-null),
// drawn[slot] (the model's own draw) when non-null, the fed-back embedding
// into ``next_in`` (nb rows), accumulates ``fsum`` and at the last level
// writes ``frame_mean`` = round(fsum / L).
void sample_level(DType dt, const float* logits, const SampleParams& p, int frame, int level, int slot,
                  const int* teacher, int* tokens, int* drawn, const void* emb, int D,
                  void* next_in, void* fsum, void* frame_mean, hipStream_t s);

// The same for `streams` independent streams in one launch (block b: logits
// rows 2b and 2b + 1, seed p.seed[b], token slots slot + b * tstride, the
// feedback rows 2b and 2b + 1 of next_in / fsum / frame_mean).  frame_ptr
// non-null: the frame index is read from it on the device and the slot
// advances by frame * rvq_depth.
// feed non-null (levels 0 .. L - 2): the fed token's row of a depth layer-0
// q/k/v table (row = token - offset, 3 HD model-dtype values q | k | v) is
// written for both rows of the stream: q into q (rows, HD), k and v into ring
// slot level + 1 of the caches kc / vc (rows, H, Lmax, 64), so the next
// level's layer 0 needs no norm or projection.  The caller passes a feed only
// when every fed token lies in the table (drawn tokens always do).
struct QkvFeed {
  const void* table = nullptr;
  void* q = nullptr;
  void* kc = nullptr;
  void* vc = nullptr;
  int HD = 0, H = 0, Lmax = 0, offset = 0, rows = 0;
};
void sample_levels(DType dt, int streams, const float* logits, const SampleParams& p, int frame,
                   const int* frame_ptr, int level, int slot, int tstride, const int* teacher, int* tokens,
                   int* drawn, const void* emb, int D, void* next_in, void* fsum, void* frame_mean, hipStream_t s,
                   const QkvFeed* feed = nullptr);

// Every level of one frame drawn at once from logits (levels, 2, C) (one
// stream, noise (F, L, C) tabulated or computed from p.seed[0]):
// drawn[l] = codec_offset + C * l + winner.
void draw_levels(const float* logits, const SampleParams& p, int frame, int levels, int* drawn, hipStream_t s);

// ---- encoder ------------------------------------------------------------------
// x[r, :] = round(emb[tok[r]] + pe_T[r % S])    (model.cpp:231-236)
void encoder_embed(DType dt, const void* emb, const void* pe, const int* tok, int M, int S,
                   int D, void* x, hipStream_t s);
// y[r, :] = rmsnorm(x[r, :]) * g   (model dtype in and out)
void rmsnorm_rows(DType dt, const void* x, const void* g, float eps, int M, int D, void* y,
                  hipStream_t s);

// GEMM C[m, n] = sum_k A[m, k] * B[n, k]; A (M, K) and B (N, K) row-major.
enum class GemmEpi : int {
  Store = 0,    // C (M, N) model dtype, ld = N
  Resid = 1,    // R[m, n] = round(R + round(acc)), ld = N
  Geglu = 2,    // B packed like gemv_geglu; C (M, N/2)
  CrossKV = 3,  // n = (layer*2 + kv)*HD + h*64 + d; m = b*S + s ->
                //   C[(((layer*2+kv)*nb + b)*H + h)*S + s][d]
  StoreF32 = 4, // C (M, N) fp32, each value rounded to the model dtype first (logits)
};
struct GemmEpiArgs {
  GemmEpi kind = GemmEpi::Store;
  void* C = nullptr;
  int nb = 2, H = 16, S = 1, HD = 1024;
};
void gemm(DType dt, const void* A, const void* B, int M, int N, int K, const GemmEpiArgs& e,
          hipStream_t s, bool allow_mfma = true);

// Bidirectional encoder self-attention, no mask, no bias, scale 1.0.
// qkv (nb*S, 3*HD) row-major [q | k | v]; out (nb*S, HD).
void encoder_attn(DType dt, const void* qkv, int nb, int S, int H, void* out, hipStream_t s,
                  bool allow_mfma = true);

// One draw as sample_level, allocating nothing: the seed and the feedback rows
// go to a fixed per-device scratch array of noalloc_scratch_bytes() bytes
// (sample_kernels.hip); the token is written to token[0].  Throws if d_model
// needs more scratch.  Calls that overlap on one device race on the scratch.
size_t noalloc_scratch_bytes();
void sample_level_noalloc(DType dt, int device, const void* emb, int D, const float* logits, const SampleParams& p,
                          uint64_t seed, int frame, int level, int* token, hipStream_t s);

// Read bandwidth (GB/s, 1e9 B/s) of `passes` reads of a `bytes` device buffer
// after one warm pass (probe_kernels.hip).
float probe_read_bandwidth(int device, size_t bytes, int passes);
// Microseconds per round of an all-gather of `words` tagged words among
// `workgroups` workgroups (one phase hand-off of the persistent kernels; `delay`
// rounds of s_sleep(1) before each round's first poll), and
// the one-way latency of a word bounced between workgroups 0 and `peer`.
float probe_handoff(int device, int workgroups, int words, int rounds, int delay);
float probe_pingpong(int device, int peer, int rounds);

}  // namespace mrt
