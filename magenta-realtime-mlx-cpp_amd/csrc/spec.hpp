// Token plumbing of speculative depth decoding (spec_kernels.hip).
#pragma once

#include "common.hpp"

namespace mrt {

// out (2L, D) rows 2i + r: the temporal output row r for i = 0, else
// emb(draft[i - 1]): the verification pass's input (decode.cpp:184-197).
void spec_inputs(DType dt, const void* t_out, const void* emb, const int* draft, int L, int D, void* out,
                 hipStream_t s);
// Accept the drafts up to the first level whose draw differs (decode.cpp:
// 225-236): tokens[0..n] = drawn[0..n], *decided = n (L: all accepted); both
// rows of next_in = emb(drawn[0]), the input of depth step 1.
void spec_accept(DType dt, const int* drawn, const int* draft, int L, int* tokens, int* decided, const void* emb,
                 int D, void* next_in, hipStream_t s);
// Frame mean of the L tokens' embeddings in the model dtype (decode.cpp:476-484), both rows.
void frame_mean_tokens(DType dt, const int* tokens, int L, const void* emb, int D, void* out, hipStream_t s);
// dst (2, C) = the logits level l was drawn from (the pass's rows 2l, 2l+1
// when l <= *decided, else slice).
void spec_record(const float* all, const float* slice, const int* decided, int l, int C, float* dst, hipStream_t s);

}  // namespace mrt
