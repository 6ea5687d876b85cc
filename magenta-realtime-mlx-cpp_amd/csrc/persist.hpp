// Persistent (one workgroup per CU) step kernels: a whole depth_step or
// temporal_step runs as ONE launch whose phases hand data to each other
// through tagged 64-bit words.  See persist_kernels.hip.
#pragma once

#include "common.hpp"
#include "kernels.hpp"

namespace mrt {

constexpr int kPersistThreads = 256;
constexpr int kMaxPersistK = 3072;  // largest GEMV input (d_model, heads*64, d_ff)
constexpr int kMaxPersistLen = 64;  // self-attention ring slots handled by the fused path
constexpr int kMaxBph = 16;         // workgroups per head
constexpr int kMaxCrossChunk = 64;  // encoder keys per workgroup in cross attention

// One decoder stack (temporal or depth) laid out per weight kind: layer i of
// a kind starts at base + i * (elements of one layer), so every address is a
// scalar function of kernel arguments.
struct DecStack {
  const void* norm_sa;  // (L, D)
  const void* wqkv;     // (L, 3 HD, D): q | k | v rows
  const void* wo;       // (L, D, HD)
  const void* norm_ca;  // (L, D)       temporal only
  const void* wq_c;     // (L, HD, D)   temporal only
  const void* wo_c;     // (L, D, HD)   temporal only
  const void* norm_ff;  // (L, D)
  const void* w01;      // (L, 2 F, D): 32-row groups [gate 32 | up 32]
  const void* wo2;      // (L, D, F)
  const void* cross;    // cross K/V: layer i K at 2i*n, V at (2i+1)*n, n = 2*H*S*64
  void* ring;           // self K/V ring: layer i K at 2i*m, V at (2i+1)*m, m = 2*H*Lmax*64
};

// Poll sites of the persistent kernels; each waits its own number of
// s_sleep(1) rounds (64 clocks each) before the first poll of its hand-off.
enum PollSite : int {
  kPollQKV = 0,     // layer input before the q/k/v projection
  kPollAttn,        // a head's q, k, v before its self attention
  kPollO,           // attention output before the output projection
  kPollCrossQ,      // layer input before the cross-attention query projection
  kPollCrossPart,   // a head's cross query before a key block's partial
  kPollCrossComb,   // the key-block partials before their combination
  kPollCrossO,      // cross-attention output before its projection
  kPollUp,          // layer input before the gated-GELU projection
  kPollDown,        // gated-GELU output before the down projection
  kPollHead,        // stack output before the head
  kPollLogits,      // head logits before the draw (workgroup 0)
  kPollToken,       // the drawn token before the next depth level
  kPollSites
};
static_assert(kPollSites <= 16, "LLBufs::delay holds 16 sites");

// Hand-off buffers of one state: 64-bit words {payload (low 32), tag (high
// 32)}.  16-bit models pack both CFG rows of an element in one payload; fp32
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
  uint64_t* tok;    // token drawn by workgroup 0 (frame kernel)
  uint32_t* seq;    // launch counter (tag epoch), advanced by each launch
  int* err;         // set when a poll exceeds its spin limit
  uint8_t delay[16];  // per PollSite: s_sleep(1) rounds before the first poll of a hand-off
};
// tag = (epoch << kTagShift) | phase code: codes stay below 1 << kTagShift,
// and the host zeroes every word and restarts the epoch at 1 before the
// epoch's low 20 bits wrap.
constexpr int kTagShift = 12;
constexpr uint32_t kEpochPeriod = 1u << (32 - kTagShift);
constexpr size_t kLLVecWords = 2 * kMaxPersistK;

struct StepArgs {
  DecStack st;
  int nlayers;
  int cross;   // temporal step (has cross attention)
  int D, HD, H, F, bph;
  int pos, Lmax;  // ring slot written this step; ring size
  const void* bias_rows;  // default self-attention bias: position p's (H, p + 1) block at H p (p + 1) / 2
  const void* bias_row;   // explicit self-attention bias (H, pos + 1) model dtype, or nullptr (bias_rows)
  const void* in;   // (2, D) model-dtype rows (plain)
  void* out;        // (2, D) rows: temporal output
  int S;            // encoder length
  // depth head
  const void* dec_norm;
  const void* head_w;  // first lm_head row of the head
  int head_rows;       // rows of the head (codebook, or vocab)
  float* logits;       // (2, head_rows) plain copy
  // sampling after the head (frame kernel)
  SampleParams sp;
  int frame;
  const int* teacher;  // (frames * levels) ids fed back instead of the draws, or nullptr
  int* tokens;         // (frames * levels) fed-back ids
  int* drawn;          // (frames * levels) drawn ids, or nullptr
  const void* emb;     // (vocab, D) token embeddings
  void* fmean;         // (2, D): frame mean (next temporal input)
  float* rec_slice;    // optional copy of the logits
  const float* noise;  // Gumbel noise of the frame's draws: (levels, codebook) floats
  LLBufs ll;
  // Optional timeline (100 MHz wall clock) recorded by workgroup 0.
  uint64_t* trace;
};
constexpr int kTraceSlots = 512;
constexpr int kTraceStart = kTraceSlots - 3;
constexpr int kTraceEnd = kTraceSlots - 2;
constexpr int kTraceDone = kTraceSlots - 1;

// Grid size of the persistent kernels for a model with H heads on this
// device (H * blocks-per-head, bph a power of two in [8, 16]); 0 if unsupported.
int persist_grid(int H, int num_cu, int* bph);

enum class PersistKernel { Temporal, Depth, Frame, Levels };
// Dynamic LDS bytes of a persistent kernel, after allowing the kernel to use
// them; 0 if the device cannot give one workgroup that much, or cannot keep
// one such workgroup resident per CU (occupancy query), in which case the
// caller uses the multi-kernel path.
size_t persist_prepare(DType dt, PersistKernel kind, int device);

// Persistent grids of different states on one device must not run at the
// same time: each takes one workgroup per CU and polls words written by the
// rest of its grid, so two grids splitting the CUs would both wait until the
// spin limit.  A PersistSection brackets the enqueue of one persistent unit of
// work (a step launch, or a whole decode: its graph launch or eager launches)
// on `stream`: it holds the device's gate mutex, makes the stream wait for the
// device's previous persistent unit (an event), and records that event after
// the enqueued work.  Units on one device therefore run one after another on
// the GPU, in the order their sections were entered, whatever host threads and
// streams enqueue them; the host does not block on the GPU.
class PersistSection {
 public:
  PersistSection(int device, hipStream_t stream);
  ~PersistSection();
  PersistSection(const PersistSection&) = delete;
  PersistSection& operator=(const PersistSection&) = delete;

 private:
  int device_;
  hipStream_t stream_;
};

void launch_step(DType dt, const StepArgs& a, int grid, size_t lds, hipStream_t s);

// One frame of the decode loop in one launch: the temporal step (t), then
// `levels` depth steps (d, d.pos ignored), each followed by a draw whose
// token is fed back on the device.  d.head_w is the first lm_head row of
// level 0's slice (level l at + l * codebook rows).
struct FrameArgs {
  StepArgs t;
  StepArgs d;
  int codebook, levels;
  float* rec_slices;   // (levels, 2, codebook) copies of the logits, or nullptr
  void* rec_temporal;  // (2, D) copy of the temporal output, or nullptr
  // Layer 0's q | k | v of every fed-back token (Model::depth_qkv_table for
  // this codebook and codec offset), or nullptr: computed at every level.
  const void* qkv_table;
  // Optional per-frame phase stamps of workgroup 0 (device wall clock):
  // [start, temporal stack done, end, ticks spent in the draws] at
  // prof + 4 * frame; nullptr: none taken.
  uint64_t* prof;
};
// The frame kernel keeps the depth K/V history in LDS: it needs
// depth layers * levels <= kMaxResidentSlots.
constexpr int kMaxResidentSlots = 64;
void launch_frame(DType dt, const FrameArgs& a, int grid, size_t lds, hipStream_t s);
// The depth levels after a speculative verification pass, in one launch:
// levels *a.d.sp.decided + 1 .. a.levels - 1 of frame a.d.frame, each a depth
// step (history staged from the ring), its head slice and a draw, as in
// launch_frame; a.t is unused and the frame mean is not formed.
void launch_levels(DType dt, const FrameArgs& a, int grid, size_t lds, hipStream_t s);

// Gumbel noise of every draw of a decode call: out[(f * L + l) * C + c] =
// gumbel(seed, f, l, c) for f < frames, l < L, c < C.
void gumbel_table(const uint64_t* seed, int frames, int L, int C, float* out, hipStream_t s);


}  // namespace mrt
