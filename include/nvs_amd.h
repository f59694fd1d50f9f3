/*
 * nvs_amd.h -- C ABI of the MI355X (gfx950) target-verify hot path of nano-vllm-speculative-decoding.
 *
 * Two ops live behind this boundary:
 *   1. paged multi-query verify attention (+ the paged KV store, and the fused q/k RMSNorm + RoPE + store, that
 *      precede it), and
 *   2. the speculative sampler: truncation -> softmax -> rejection test -> residual / bonus race.
 * Two elementwise ops of the decoder layer (RMSNorm with the residual add, SiLU-and-mul) complete a verify forward
 * around the library GEMMs.
 *
 * Every entry point takes plain device pointers, element strides and sizes, plus the HIP stream to launch on
 * (NULL = the legacy default stream). Nothing here allocates, synchronises the host with the device, or reads a
 * device value on the host, so every call is safe inside HIP-graph capture when its workspace is preallocated.
 *
 * Return value: NVS_OK (0) or a negative nvs_status. On failure nvs_last_error() returns a message describing it
 * (thread-local; valid until the next call on the same thread). Argument errors are detected on the host before any
 * launch, so they are testable without a GPU.
 *
 * Strides are in ELEMENTS, not bytes. Token ids, lengths and counts follow the reference's dtypes: int32 for the
 * attention metadata (cu_seqlens, context_lens, block_tables, slot_mapping), int64 for drafts, top_k,
 * verified_lens and the sampler outputs.
 */
#ifndef NVS_AMD_H
#define NVS_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NVS_ABI_VERSION 9

typedef enum {
    NVS_OK = 0,
    NVS_ERR_INVALID = -1,      /* bad argument: shape, stride, alignment, null pointer */
    NVS_ERR_UNSUPPORTED = -2,  /* valid for the reference but not implemented by this library (e.g. head_dim 96) */
    NVS_ERR_WORKSPACE = -3,    /* workspace missing or smaller than the matching *_workspace_size */
    NVS_ERR_HIP = -4           /* the HIP runtime reported an error at launch */
} nvs_status;

typedef enum {
    NVS_DTYPE_F32 = 0,
    NVS_DTYPE_BF16 = 1,
    NVS_DTYPE_F16 = 2
} nvs_dtype;

/* Version of this header's ABI; the Python loader refuses a library whose version differs. */
int nvs_abi_version(void);

/* Message of the last failed call on this thread ("" when none). */
const char* nvs_last_error(void);

/* ------------------------------------------------------------------------------------------------ KV store
 * Replaces store_kvcache / store_kvcache_kernel (nanovllm/layers/attention.py:10-40; semantics restated in
 * tests/fake_paged_attention.py:14-17).
 * Cache geometry (shared by every entry point that writes the cache): both caches are
 * [cache_blocks, block_size, n_kv_heads, head_dim] with element strides cache_block_stride, cache_token_stride,
 * cache_head_stride and a contiguous head_dim; slot s is token s % block_size of block s / block_size. The
 * reference's token-major layout (model_runner.py:160) has strides (block_size*n_kv_heads*head_dim,
 * n_kv_heads*head_dim, head_dim); a head-major cache [cache_blocks, n_kv_heads, block_size, head_dim], in which the
 * attention streams each (block, head) as one contiguous run, has (n_kv_heads*block_size*head_dim, head_dim,
 * block_size*head_dim).
 * For i < n_tokens with s = slot_mapping[i] >= 0 (the reference skips exactly s == -1; negative slots and slots
 * >= cache_blocks*block_size are skipped here too instead of writing out of bounds), for every head h and e < head_dim:
 *   k_cache[block(s), token(s), h, e] = key[i*key_row_stride + h*head_dim + e], and v_cache likewise from value.
 * Each token row of key/value must be contiguous (the reference asserts stride(-1) == 1 and stride(1) == head_dim);
 * value may be a strided view (a slice of the fused qkv output). A pure copy: bit-exact for every dtype. */
int nvs_store_kvcache(const void* key, int64_t key_row_stride,
                      const void* value, int64_t value_row_stride,
                      void* k_cache, void* v_cache, int64_t cache_blocks, int64_t block_size,
                      int64_t cache_block_stride, int64_t cache_token_stride, int64_t cache_head_stride,
                      const int32_t* slot_mapping, int64_t n_tokens,
                      int n_kv_heads, int head_dim, int dtype, void* stream);

/* ------------------------------------------------------------------------------------------------ q/k norm, RoPE, store
 * Replaces the sequence between the qkv projection and the attention kernel, in one launch:
 *   q = q_norm(q); k = k_norm(k); q, k = rotary_emb(positions, q, k)   (nanovllm/models/qwen3.py:82-85;
 *   RMSNorm.rms_forward nanovllm/layers/layernorm.py:15-24; apply_rotary_emb / RotaryEmbedding.forward
 *   nanovllm/layers/rotary_embedding.py:6-14,37-47), then store_kvcache(k, v, k_cache, v_cache, slot_mapping)
 *   (Attention.forward, nanovllm/layers/attention.py:63-64).
 * With n_heads == 0 and q = q_out = NULL it is the draft model's keys-only path (DFlashDraftModel.store_context_kv,
 * nanovllm/models/dflash.py:88-96: k_norm, apply_rotary_emb_k, store_kvcache).
 * Per token t and head h (head_dim D = 128, neox halves x1 = x[:64], x2 = x[64:]):
 *   RMSNorm (when the head's weight is non-NULL): y = dtype(float(x) / sqrt(mean(float(x)^2) + eps)), then
 *   y = dtype(float(y) * float(weight)); rotary: with c = cos_sin_cache[p, :64], s = cos_sin_cache[p, 64:] and
 *   p = positions[t] (clamped into [0, cache_positions)), o = dtype(concat(y1*c - y2*s, y2*c + y1*s)), every
 *   product and sum rounded separately as in the eager ops.
 * q_out[t, h] = o for query heads (q_out may alias q); for key heads o goes to k_out (when non-NULL) and, like v, to
 * cache slot slot_mapping[t] (skipped when negative or >= cache_blocks*block_size, as store_kvcache skips -1).
 * q, k, v, q_out, k_out: [n_tokens, heads, 128] with the given token strides and head stride 128 (views of the fused
 * qkv output are fine); weights [128] in the same dtype; cos_sin_cache [cache_positions, 128] fp32 (the
 * reference's cos_sin_cache buffer); caches of the cache geometry described at nvs_store_kvcache. dtype bf16 or
 * fp16. */
int nvs_qk_norm_rope_store(const void* q, int64_t q_token_stride, const void* k, int64_t k_token_stride,
                           const void* v, int64_t v_token_stride, const int64_t* positions,
                           const void* q_norm_weight, const void* k_norm_weight, float eps,
                           const float* cos_sin_cache, int64_t cache_positions,
                           const int32_t* slot_mapping, void* k_cache, void* v_cache, int64_t cache_blocks,
                           int64_t block_size, int64_t cache_block_stride, int64_t cache_token_stride,
                           int64_t cache_head_stride,
                           void* q_out, int64_t q_out_token_stride, void* k_out, int64_t k_out_token_stride,
                           int64_t n_tokens, int n_heads, int n_kv_heads, int head_dim, int dtype, void* stream);

/* ------------------------------------------------------------------------------------------------ attention
 * Replaces both flash-attn calls of Attention.forward (nanovllm/layers/attention.py:59-77):
 *   varlen mode  (cu_seqlens_q and cu_seqlens_k non-NULL) = flash_attn_varlen_func(..., causal=True,
 *                block_table=block_tables) of the verify / cached-prefix branch (attention.py:64-70);
 *   fixed mode   (both NULL, context_lens non-NULL)      = flash_attn_with_kvcache(q.view(-1, query_len_per_seq, H,
 *                D), cache_seqlens=context_lens, causal=causal) of the decode / draft-block branch (attention.py:71-76).
 * Row r owns Lq query tokens starting at token q0 (varlen: q0 = cu_seqlens_q[r], Lq = cu_seqlens_q[r+1]-q0;
 * fixed: q0 = r*query_len_per_seq, Lq = query_len_per_seq) and Lk keys (cu_seqlens_k[r+1]-cu_seqlens_k[r] or
 * context_lens[r]); key j lives at k_cache[block_tables[r*bt_row_stride + j/block_size], j%block_size, g].
 * Query i (< Lq) of head h attends to keys j < Lk, and with causal only to j <= Lk - Lq + i (bottom-right
 * alignment), through kv head g = h / (n_heads/n_kv_heads):
 *   out[q0+i, h] = softmax_j(scale * q[q0+i, h] . K_j) V_j, fp32 softmax and accumulation, bf16 out.
 * Rows with Lq = 0 write nothing; a query that sees no key gets zeros.
 * q and out are [n_tokens, n_heads, head_dim] with the given token/head strides; both caches share the strides
 * [blocks, block_size, n_kv_heads, head_dim]. Supported here: dtype bf16, head_dim 128, block_size a multiple of 32,
 * (n_heads/n_kv_heads)*max_seqlen_q any size (packed into 32-row tiles). max_seqlen_k bounds every Lk (the graph
 * capture passes max_model_len); the grid depends only on the host integers, so a captured launch stays valid for
 * any device lengths within those bounds.
 * workspace: device memory of at least nvs_paged_attention_workspace_size(...) bytes (may be NULL when that is 0);
 * no initialisation needed. One launch: when the plan splits a row's keys, each split writes an fp32 partial to
 * the workspace and the (row, kv head, query tile) unit's last split to finish merges them. unit_counters: int32
 * [n_rows * n_kv_heads * ceil((n_heads/n_kv_heads) * max_seqlen_q / 32)] device buffer that is zero on entry;
 * every call leaves it zero again (keep one zero-filled buffer and reuse it; calls sharing it must be ordered on
 * one stream). It may be NULL when the workspace size is 0 (no split).
 * Bounds: n_tokens (rows of q / out), cache_blocks (blocks of each cache) and bt_width (valid entries per block
 * table row) bound every index the kernel derives from device metadata; inconsistent metadata gives wrong
 * numbers for the rows concerned, never an access outside the buffers. */
int nvs_paged_attention_workspace_size(int n_rows, int n_heads, int n_kv_heads, int head_dim,
                                       int max_seqlen_q, int max_seqlen_k, size_t* bytes);

int nvs_paged_attention(const void* q, int64_t q_token_stride, int64_t q_head_stride, int64_t n_tokens,
                        const void* k_cache, const void* v_cache, int64_t cache_blocks,
                        int64_t cache_block_stride, int64_t cache_token_stride, int64_t cache_head_stride,
                        const int32_t* block_tables, int64_t bt_row_stride, int bt_width,
                        const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                        const int32_t* context_lens, int query_len_per_seq,
                        int n_rows, int max_seqlen_q, int max_seqlen_k,
                        int n_heads, int n_kv_heads, int head_dim, int block_size,
                        float scale, int causal, int dtype,
                        void* out, int64_t out_token_stride, int64_t out_head_stride,
                        int32_t* unit_counters, void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------------------------------ sampler
 * Shared conventions (nanovllm/layers/spec_sampler.py):
 *   logits are [n_pos, V] rows with row stride logits_row_stride, dtype f32/bf16/f16, upcast to fp32;
 *   per-row sampling parameters (SamplingTensors, spec_sampler.py:17-24) are indexed by param row
 *   pos / pos_per_param: temperatures f32 (divided into the logits, IEEE division), top_k int64 (0 = off),
 *   top_p f32 (1 = off); max_top_k and has_top_p are the host flags of SamplingTensors.
 *   Truncation = truncate_logits (spec_sampler.py:72-96): keep s >= threshold, ties kept, HuggingFace order
 *   temperature -> top-k -> top-p-within-top-k; probabilities = softmax over the kept set.
 * Any max_top_k >= 0 (top_k up to the vocabulary, sampling_params.py:15-16); windows wider than 1024 values take a
 * slower exact path over the row. nvs_markov_draw alone is limited to max_top_k <= 1024 (NVS_ERR_UNSUPPORTED). */

/* probs_from_logits (spec_sampler.py:65-69): dense fp32 probabilities [n_pos, V] into probs (row stride V). */
int nvs_probs_from_logits_workspace_size(int64_t n_pos, int64_t vocab, int max_top_k, size_t* bytes);
int nvs_probs_from_logits(const void* logits, int logits_dtype, int64_t logits_row_stride,
                          int64_t n_pos, int64_t vocab, int64_t pos_per_param,
                          const float* temperatures, const int64_t* top_k, const float* top_p,
                          int max_top_k, int has_top_p,
                          float* probs, void* workspace, size_t workspace_bytes, void* stream);

/* truncate_logits (spec_sampler.py:72-96) of already temperature-scaled fp32 logits: out = scaled, or -inf below
 * each row's threshold. out may alias scaled. */
int nvs_truncate_logits(const float* scaled, int64_t scaled_row_stride, int64_t n_pos, int64_t vocab,
                        int64_t pos_per_param, const int64_t* top_k, const float* top_p,
                        int max_top_k, int has_top_p,
                        float* out, void* workspace, size_t workspace_bytes, void* stream);

/* race / sample (spec_sampler.py:99-111): out[r] = argmax_i weights[r,i] / noise[r,i] (first index wins ties),
 * weights and noise fp32 [n_rows, V] with the given row strides.
 * One launch over (row, vocabulary chunk) workgroups: the last chunk of each row to finish picks the row's winner.
 * row_counters: int32 [n_rows] device buffer that is zero on entry; every call leaves it zero again (keep one
 * zero-filled buffer and reuse it; calls sharing it must be ordered on one stream). workspace: scratch of
 * nvs_race_workspace_size bytes, no initialisation needed. */
int nvs_race(const float* weights, int64_t weights_row_stride, const float* noise, int64_t noise_row_stride,
             int64_t n_rows, int64_t vocab, int64_t* out, int32_t* row_counters, void* workspace,
             size_t workspace_bytes, void* stream);
int nvs_race_workspace_size(int64_t n_rows, int64_t vocab, size_t* bytes);

/* accept_random_varlen (spec_sampler.py:123-150) over dense probabilities, with the generator's draws passed in:
 * uniforms = torch.rand(B, k) and noise = exponential_noise_([B, V]) drawn in that order by the caller.
 * p [T, V] fp32 (row stride V), q [B, k, V] fp32 contiguous, drafts [B, k] int64, verified_lens [B] int64 in
 * 1..k+1 summing to T (NULL = every row verifies k+1 = accept_random, spec_sampler.py:114-120).
 * Outputs n_accept [B] int64 and tail [B] int64. One launch, like nvs_race; row_counters: int32 [B], zero on
 * entry and left zero, as for nvs_race. */
int nvs_accept_random_workspace_size(int64_t batch, int64_t vocab, size_t* bytes);
int nvs_accept_random(const float* p, const float* q, const int64_t* drafts, const int64_t* verified_lens,
                      const float* uniforms, const float* noise,
                      int64_t batch, int num_drafts, int64_t n_pos, int64_t vocab,
                      int64_t* n_accept, int64_t* tail, int32_t* row_counters, void* workspace,
                      size_t workspace_bytes, void* stream);

/* accept_greedy_varlen (spec_sampler.py:153-169): target tokens = argmax of each logit row (first max wins);
 * a draft is accepted iff it equals the target token at its position; tail = the target token after the
 * accepted prefix. verified_lens NULL = every row verifies k+1 (accept_greedy). */
int nvs_accept_greedy_workspace_size(int64_t n_pos, int64_t vocab, size_t* bytes);
int nvs_accept_greedy(const void* logits, int logits_dtype, int64_t logits_row_stride,
                      const int64_t* drafts, const int64_t* verified_lens,
                      int64_t batch, int num_drafts, int64_t n_pos, int64_t vocab,
                      int64_t* n_accept, int64_t* tail, void* workspace, size_t workspace_bytes, void* stream);

/* The fused verify sampler: probs_from_logits(logits, sampling_per_token(...)) followed by accept_random_varlen
 * (the two calls SpeculativeDecoder._accept makes, nanovllm/engine/speculative.py:450-462), in one pass over each
 * verified position's logit row. The [T, V] probabilities are never written: each position's kept set (top-k
 * window plus ties, then top-p) is selected on chip, the accept test reads p and q at the draft token only, and
 * the residual max(p - q, 0) or bonus race reads q and the noise only inside the kept set (a row with top_k = 0
 * falls back to a full-vocabulary race). Same outputs as the two calls given the same uniforms and noise.
 * Sampling parameters are per batch row [B] (not per token). verified_lens must sum to n_pos, as the reference
 * requires (spec_sampler.py:127-129).
 * One launch: the last position of each batch row to finish counts the row's accepted prefix and writes its
 * outputs. row_counters: int32 [batch] device buffer that is zero on entry; every call leaves it zero again, so a
 * caller keeps one zero-filled buffer and reuses it (calls sharing it must be ordered on one stream).
 * workspace: scratch of nvs_spec_accept_workspace_size bytes, no initialisation needed. */
int nvs_spec_accept_workspace_size(int64_t batch, int num_drafts, int64_t n_pos, int64_t vocab, int max_top_k,
                                   size_t* bytes);
int nvs_spec_accept(const void* logits, int logits_dtype, int64_t logits_row_stride,
                    const float* temperatures, const int64_t* top_k, const float* top_p,
                    int max_top_k, int has_top_p,
                    const float* q, const int64_t* drafts, const int64_t* verified_lens,
                    const float* uniforms, const float* noise,
                    int64_t batch, int num_drafts, int64_t n_pos, int64_t vocab,
                    int64_t* n_accept, int64_t* tail, int32_t* row_counters,
                    void* workspace, size_t workspace_bytes, void* stream);

/* nvs_spec_accept with the draft q as candidate rows (the sparse rows nvs_markov_draw writes) instead of a dense
 * [batch, num_drafts, vocab] tensor: q[b, j, v] = cand_probs[(b * num_drafts + j) * cand_row_stride + c] where
 * cand_ids[...same...] == v (c < num_candidates; id -1 holds no token), else 0. The same decisions as
 * nvs_spec_accept on the scattered q (the reference's draft_probs, speculative.py:169-180). Every row truncates
 * with top-k (max_top_k >= 1; a row with top_k <= 0 is treated as top-k max_top_k), as DSpark's candidate batches
 * do. */
int nvs_spec_accept_candidates(const void* logits, int logits_dtype, int64_t logits_row_stride,
                               const float* temperatures, const int64_t* top_k, const float* top_p, int max_top_k,
                               int has_top_p, const int32_t* cand_ids, const float* cand_probs, int num_candidates,
                               int64_t cand_row_stride, const int64_t* drafts, const int64_t* verified_lens,
                               const float* uniforms, const float* noise, int64_t batch, int num_drafts,
                               int64_t n_pos, int64_t vocab, int64_t* n_accept, int64_t* tail,
                               int32_t* row_counters, void* workspace, size_t workspace_bytes, void* stream);

/* nvs_spec_accept with no workspace and no row counters from the caller. It has no counterpart in the reference:
 * it is for callers that cannot allocate device memory (code under HIP graph capture, serving loops or harnesses
 * that forbid allocation). The records, dense-race state and per-row counters live in a fixed device array of the
 * library (1 MiB + 4 KiB per device, held until the process ends), resolved per device on the first call.
 * Same arguments and results as nvs_spec_accept otherwise. Limits: batch <= 1024 and at most 1 MiB of records
 * (32 bytes per verify position, plus the dense races' state when max_top_k == 0); larger calls return
 * NVS_ERR_UNSUPPORTED before any launch. All calls on one device share the array: calls that overlap on a device
 * (other streams, other host threads) race; calls ordered on one stream do not. Each call clears its row counters
 * with a kernel first (no memset node, so it can be captured). */
int nvs_spec_accept_noalloc(const void* logits, int logits_dtype, int64_t logits_row_stride,
                            const float* temperatures, const int64_t* top_k, const float* top_p, int max_top_k,
                            int has_top_p, const float* q, const int64_t* drafts, const int64_t* verified_lens,
                            const float* uniforms, const float* noise, int64_t batch, int num_drafts,
                            int64_t n_pos, int64_t vocab, int64_t* n_accept, int64_t* tail, void* stream);

/* ------------------------------------------------------------------------------------------------ Markov draw
 * Replaces one candidate row of DFlashDrafter._markov_rows (nanovllm/engine/speculative.py:163-184, the
 * `elif candidates:` branch): for each of `batch` sequences,
 *   row_logits = dtype(logits[b] + bias[b])                    (bias: the row's Markov bias, markov_head(prev);
 *                                                               NULL when the caller added it already)
 *   values, ids = topk(row_logits, num_candidates)            (ties in index order)
 *   probs = probs_from_logits(values, sampling)                (temperature, top-k, top-p over the candidates)
 *   token = ids[race(probs, noise[:, row])]                    (argmax of probs / noise, first rank on ties)
 * and writes the sparse row instead of scattering it over the vocabulary: cand_ids[b, c] / cand_probs[b, c] for
 * the candidates with a non-zero probability, in rank order, then id -1 and probability 0 up to num_candidates;
 * draws[b * draws_stride] = token. Only the kept candidates are ranked: the others have probability 0 in the
 * reference and never win its race unless every probability is 0 (then rank 0, the row's largest value).
 * num_candidates is the reference's num_candidates() = min(max_top_k + 64, vocab); every row must truncate with
 * top-k (the reference's candidate rows require it; a row with top_k <= 0 is drawn among its top max_top_k).
 * logits and bias [batch, vocab] fp32 / bf16 / fp16 (one dtype) with row strides; noise [batch, >= num_candidates]
 * fp32, the row's exponential noise by candidate rank; parameters per row as in nvs_probs_from_logits.
 * min(max_top_k, vocab) <= num_candidates <= 7168; batch <= 65535. With at most 512 candidates, at most 64
 * segments of up to 19,456 values (a vocabulary up to 1,245,184) and segments x candidates <= 4,096, the row is
 * cut into segments drawn by separate workgroups of one launch, and the row's last segment to finish merges them
 * (workspace: nvs_markov_draw_workspace_size bytes, no initialisation; row_counters: int32 [batch], zero on the
 * first call and left zero by every call, shared only by calls ordered on one stream); otherwise one workgroup
 * draws each row, needs no workspace or counters, and takes no bias (add it first).
 * The rows of a draft block are sequential launches because each row's bias depends on the token drawn before it. */
int nvs_markov_draw_workspace_size(int64_t batch, int64_t vocab, int num_candidates, size_t* bytes);
int nvs_markov_draw(const void* logits, int logits_dtype, int64_t logits_row_stride, const void* bias,
                    int64_t bias_row_stride, int64_t batch, int64_t vocab, const float* temperatures,
                    const int64_t* top_k, const float* top_p, int max_top_k, int has_top_p, int num_candidates,
                    const float* noise, int64_t noise_row_stride, int32_t* cand_ids, float* cand_probs,
                    int64_t cand_row_stride, int64_t* draws, int64_t draws_stride, int32_t* row_counters,
                    void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------------ decoder-layer elementwise ops
 * The elementwise steps between the projections of a Qwen3 decoder layer, so that a whole verify forward runs
 * on this library and the GEMMs (Qwen3DecoderLayer.forward, nanovllm/models/qwen3.py:146-160).
 *
 * nvs_rms_norm replaces RMSNorm.forward (nanovllm/layers/layernorm.py:15-46). Per row:
 *   x' = float(x) (+ float(residual) when residual is non-NULL, and then residual = dtype(x'), written in place);
 *   out = dtype(dtype(x' / sqrt(mean(x'^2) + eps)) * weight)   (the reference's explicit casts, one rounding each).
 * x, residual, out: [n_rows, hidden] with the given row strides; weight [hidden]; dtype bf16 or fp16; hidden a
 * multiple of 8, at most 8192; pointers 16-byte aligned and row strides multiples of 8 (NVS_ERR_UNSUPPORTED
 * otherwise). out may alias x, not residual. The sum of squares is an fp32 sum in a fixed order. */
int nvs_rms_norm(const void* x, int64_t x_row_stride, void* residual, int64_t residual_row_stride,
                 const void* weight, float eps, void* out, int64_t out_row_stride, int64_t n_rows, int hidden,
                 int dtype, void* stream);

/* nvs_silu_and_mul replaces SiluAndMul.forward (nanovllm/layers/activation.py:8-11): per row of x = [gate | up],
 * each of width elements, out = dtype(silu(gate) * up), computed in fp32 and rounded once (the reference runs it
 * under torch.compile, which keeps the product in fp32). x [n_rows, 2 * width], out [n_rows, width]; dtype bf16 or
 * fp16; width a multiple of 8; pointers 16-byte aligned and row strides multiples of 8. */
int nvs_silu_and_mul(const void* x, int64_t x_row_stride, void* out, int64_t out_row_stride, int64_t n_rows,
                     int width, int dtype, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* NVS_AMD_H */
