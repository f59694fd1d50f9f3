// The fused accept (spec_sampler.hip) as other translation units of the library launch it.
#pragma once

#include <cstddef>
#include <cstdint>

namespace nvs {

// Workspace bytes of one fused accept over a dense q: a record per verify position, and when no row truncates
// (max_top_k == 0) the state of the dense races that follow the accept kernel.
size_t spec_accept_workspace_bytes(int64_t batch, int64_t n_pos, int64_t vocab, int max_top_k);

// nvs_spec_accept's work after its error state is cleared: argument checks, then the launches on `stream`.
int spec_accept_dense_q(const void* logits, int logits_dtype, int64_t logits_row_stride, const float* temperatures,
                        const int64_t* top_k, const float* top_p, int max_top_k, int has_top_p, const float* q,
                        const int64_t* drafts, const int64_t* verified_lens, const float* uniforms,
                        const float* noise, int64_t batch, int num_drafts, int64_t n_pos, int64_t vocab,
                        int64_t* n_accept, int64_t* tail, int32_t* row_counters, void* workspace,
                        size_t workspace_bytes, void* stream);

}  // namespace nvs
