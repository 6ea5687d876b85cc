// Persistent (one workgroup per CU) step kernels: a whole depth_step or
// temporal_step runs as ONE launch whose phases hand data to each other
// through tagged 64-bit words.  See persist_kernels.hip.
#pragma once

#include "common.hpp"
#include "kernels.hpp"

namespace mrt {

constexpr int kPersistThreads = 256;
constexpr int kMaxPersistK = 3072;  // largest GEMV input (d_model, heads*64, d_ff)
constexpr int kMaxPersistLen = 64;  // self-attention keys handled by the fused path
constexpr int kMaxBph = 16;         // workgroups per head

// Per-layer device pointers (weights of the model + this state's caches).
struct LayerDev {
  const void* norm_sa;
  const void* wqkv;
  const void* wo;
  const void* norm_ca;
  const void* wq_c;
  const void* wo_c;
  const void* norm_ff;
  const void* w01;
  const void* wo2;
  const void* ck;  // cross K (rows, H, S, 64)
  const void* cv;
  void* kc;        // self K ring (rows, H, Lmax, 64)
  void* vc;
};

// Hand-off buffers of one state: 64-bit words {payload (low 32), tag (high
// 32)}.  bf16 models pack both CFG rows of an element in one payload; fp32
// models use one word per row, row 1 at +kMaxPersistK.
struct LLBufs {
  uint64_t* x;      // residual stream (2 * kMaxPersistK words)
  uint64_t* q;      // q / cross q
  uint64_t* k;      // new K slot
  uint64_t* v;      // new V slot
  uint64_t* at;     // attention output
  uint64_t* h;      // gated-GELU output
  uint64_t* part;   // cross-attention partials: H * kMaxBph * 2 * 66 words
  uint64_t* logit;  // head logits: 2 * head_rows words
  uint32_t* seq;    // launch counter (tag epoch), advanced by each launch
  int* err;         // set when a poll exceeds its spin limit
};
constexpr size_t kLLVecWords = 2 * kMaxPersistK;

struct StepArgs {
  const LayerDev* layers;
  int nlayers;
  int cross;   // temporal step (has cross attention)
  int D, HD, H, F, bph;
  int pos, Lmax;  // ring slot written this step; ring size
  const void* bias_tab;
  const int* buckets;
  const void* in;   // (D) row pairs (plain)
  void* out;        // (D) row pairs (plain): temporal output
  int S;            // encoder length
  // depth head
  const void* dec_norm;
  const void* head_w;  // first lm_head row of the head
  int head_rows;       // rows of the head (codebook, or vocab)
  float* logits;       // (2, head_rows) plain copy
  // sampling after the head (depth step of the decode loop)
  int do_sample;
  SampleParams sp;
  int frame, level, slot;
  const int* teacher;
  int* tokens;
  int* drawn;
  const void* emb;
  void* next_in;   // (D) pairs: embedding of the fed-back token
  void* fsum;      // (D) pairs
  void* fmean;     // (D) pairs: frame mean (next temporal input)
  float* rec_slice;  // optional copy of the logits
  LLBufs ll;
  // Optional phase timeline (100 MHz wall clock) recorded by workgroup 0.
  uint64_t* trace;
};
constexpr int kTraceSlots = 512;
constexpr int kTraceStart = kTraceSlots - 3;
constexpr int kTraceEnd = kTraceSlots - 2;
constexpr int kTraceDone = kTraceSlots - 1;

// Grid size of the persistent kernels for a model with H heads on this
// device (H * blocks-per-head, bph a power of two in [8, 16]); 0 if unsupported.
int persist_grid(int H, int num_cu, int* bph);

void launch_step(DType dt, const StepArgs& a, int grid, hipStream_t s);

// (rows=2, D) model-dtype rows <-> (D) pairs.
void rows_to_pairs(DType dt, const void* rows, int D, void* pairs, hipStream_t s);
void pairs_to_rows(DType dt, const void* pairs, int D, void* rows, hipStream_t s);
// pairs[d] = (emb[id, d], emb[id, d])
void embed_pairs(DType dt, const void* emb, int D, int id, void* pairs, hipStream_t s);

}  // namespace mrt
