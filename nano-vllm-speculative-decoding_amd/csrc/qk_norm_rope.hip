// Fused per-head RMSNorm of q and k, rotary embedding of both, and the paged KV store, in one launch.
// Reference (the sequence it replaces, for a layer whose qkv projection has no bias):
//   Qwen3Attention.forward, nanovllm/models/qwen3.py:77-86      q = q_norm(q); k = k_norm(k); q, k = rotary_emb(...)
//   RMSNorm.rms_forward, nanovllm/layers/layernorm.py:15-24       per head over head_dim, eps, weight in the dtype
//   apply_rotary_emb / RotaryEmbedding.forward,
//       nanovllm/layers/rotary_embedding.py:6-14,37-47           neox halves, cos/sin from cos_sin_cache[positions]
//   Attention.forward -> store_kvcache, nanovllm/layers/attention.py:59-64
// and the keys-only variant of the draft model (DFlashDraftModel.store_context_kv, nanovllm/models/dflash.py:88-96:
// k_norm, apply_rotary_emb_k, store_kvcache; no queries).
//
// One wavefront per (token, head row); head rows are the Hq query heads, then the Hkv key heads, then the Hkv
// value heads of the token. With head_dim 128, lane l holds elements l and l + 64: exactly the pair the rotation
// mixes, so the whole op is lane-local apart from the sum of squares (one DPP reduction).
//
// Every step follows the eager op order and rounding of the reference, element by element:
//   xf = float(x); var = mean(xf^2); xf *= 1 / sqrt(var + eps)    (correctly rounded sqrt and division)
//   y = dtype(xf); y = dtype(float(y) * float(w))                   (x.to(orig_dtype).mul_(weight))
//   o1 = float(y1) * cos - float(y2) * sin; o2 = float(y2) * cos + float(y1) * sin, each product and sum rounded
//   separately (contraction off); out = dtype(o)
// The only difference from torch's CPU path is the summation order of the 128 squares.
#include "nvs_common.hpp"

namespace {

constexpr int kHeadDim = 128;
constexpr int kHalf = kHeadDim / 2;
constexpr int kRowsPerBlock = 4;  // head rows (one per wavefront) per 256-thread workgroup

struct NormRopeArgs {
    const uint16_t* q;
    int64_t q_ts;
    const uint16_t* k;
    int64_t k_ts;
    const uint16_t* v;
    int64_t v_ts;
    const int64_t* pos;
    const uint16_t* qw;
    const uint16_t* kw;
    float eps;
    const float* cs;       // [n_cs, head_dim]: cos at [0, 64), sin at [64, 128)
    int64_t n_cs;
    const int32_t* slots;  // [T], < 0: not stored
    nvs::CacheGeometry geo;  // of kc and vc (element strides)
    uint16_t* kc;
    uint16_t* vc;
    uint16_t* qo;          // [T, Hq, head_dim]
    int64_t qo_ts;
    uint16_t* ko;          // [T, Hkv, head_dim] or null
    int64_t ko_ts;
    int hq, hkv;
};

template <int DT>
__device__ __forceinline__ float to_f(uint16_t b) {
    if constexpr (DT == NVS_DTYPE_BF16) {
        return nvs::bf16_bits_to_float(b);
    } else {
        return nvs::f16_bits_to_float(b);
    }
}

template <int DT>
__device__ __forceinline__ uint16_t to_bits(float f) {
    if constexpr (DT == NVS_DTYPE_BF16) {
        return nvs::float_to_bf16_bits(f);
    } else {
        return __half_as_ushort(__float2half_rn(f));
    }
}

template <int DT>
__global__ __launch_bounds__(64 * kRowsPerBlock) void qk_norm_rope_store_kernel(NormRopeArgs a) {
#pragma clang fp contract(off)
    const int64_t t = blockIdx.x;
    const int row = static_cast<int>(blockIdx.y) * kRowsPerBlock + static_cast<int>(threadIdx.x >> 6);
    const int l = threadIdx.x & 63;
    if (row >= a.hq + 2 * a.hkv) return;  // the whole wavefront
    const int32_t slot = a.slots != nullptr ? a.slots[t] : -1;
    const bool store = slot >= 0 && slot < a.geo.slots();
    if (row >= a.hq + a.hkv) {  // value head: a copy into the cache
        const int h = row - a.hq - a.hkv;
        if (store) {
            const uint16_t* src = a.v + t * a.v_ts + static_cast<int64_t>(h) * kHeadDim;
            uint16_t* dst = a.vc + a.geo.offset(slot, h);
            dst[l] = src[l];
            dst[l + kHalf] = src[l + kHalf];
        }
        return;
    }
    const bool is_q = row < a.hq;
    const int h = is_q ? row : row - a.hq;
    const uint16_t* src = is_q ? a.q + t * a.q_ts + static_cast<int64_t>(h) * kHeadDim
                               : a.k + t * a.k_ts + static_cast<int64_t>(h) * kHeadDim;
    float x1 = to_f<DT>(src[l]);
    float x2 = to_f<DT>(src[l + kHalf]);
    const uint16_t* w = is_q ? a.qw : a.kw;
    if (w != nullptr) {
        const float sq1 = x1 * x1;
        const float sq2 = x2 * x2;
        const float var = nvs::wave_sum(sq1 + sq2) * (1.0f / kHeadDim);  // exact scaling by 2^-7
        const float r = 1.0f / sqrtf(var + a.eps);
        x1 = to_f<DT>(to_bits<DT>(x1 * r));
        x2 = to_f<DT>(to_bits<DT>(x2 * r));
        x1 = to_f<DT>(to_bits<DT>(x1 * to_f<DT>(w[l])));
        x2 = to_f<DT>(to_bits<DT>(x2 * to_f<DT>(w[l + kHalf])));
    }
    int64_t p = a.pos[t];
    p = p < 0 ? 0 : (p >= a.n_cs ? a.n_cs - 1 : p);  // out-of-table positions are clamped, never read past it
    const float c = a.cs[p * kHeadDim + l];
    const float s = a.cs[p * kHeadDim + kHalf + l];
    const float c1 = x1 * c;
    const float s2 = x2 * s;
    const float c2 = x2 * c;
    const float s1 = x1 * s;
    const uint16_t o1 = to_bits<DT>(c1 - s2);
    const uint16_t o2 = to_bits<DT>(c2 + s1);
    if (is_q) {
        uint16_t* dst = a.qo + t * a.qo_ts + static_cast<int64_t>(h) * kHeadDim;
        dst[l] = o1;
        dst[l + kHalf] = o2;
        return;
    }
    if (a.ko != nullptr) {
        uint16_t* dst = a.ko + t * a.ko_ts + static_cast<int64_t>(h) * kHeadDim;
        dst[l] = o1;
        dst[l + kHalf] = o2;
    }
    if (store) {
        uint16_t* dst = a.kc + a.geo.offset(slot, h);
        dst[l] = o1;
        dst[l + kHalf] = o2;
    }
}

}  // namespace

extern "C" int nvs_qk_norm_rope_store(const void* q, int64_t q_token_stride, const void* k, int64_t k_token_stride,
                                      const void* v, int64_t v_token_stride, const int64_t* positions,
                                      const void* q_norm_weight, const void* k_norm_weight, float eps,
                                      const float* cos_sin_cache, int64_t cache_positions,
                                      const int32_t* slot_mapping, void* k_cache, void* v_cache,
                                      int64_t cache_blocks, int64_t block_size, int64_t cache_block_stride,
                                      int64_t cache_token_stride, int64_t cache_head_stride,
                                      void* q_out, int64_t q_out_token_stride, void* k_out,
                                      int64_t k_out_token_stride, int64_t n_tokens, int n_heads, int n_kv_heads,
                                      int head_dim, int dtype, void* stream) {
    nvs::clear_error();
    NVS_CHECK(dtype == NVS_DTYPE_BF16 || dtype == NVS_DTYPE_F16, NVS_ERR_UNSUPPORTED,
              "qk_norm_rope_store: dtype %d unsupported (bf16 or fp16)", dtype);
    NVS_CHECK(head_dim == kHeadDim, NVS_ERR_UNSUPPORTED, "qk_norm_rope_store: head_dim %d unsupported (only 128)",
              head_dim);
    NVS_CHECK(n_tokens >= 0 && n_heads >= 0 && n_kv_heads > 0, NVS_ERR_INVALID,
              "qk_norm_rope_store: bad sizes n_tokens=%lld n_heads=%d n_kv_heads=%d", (long long)n_tokens, n_heads,
              n_kv_heads);
    if (n_tokens == 0) return NVS_OK;
    NVS_CHECK(k && v && positions && cos_sin_cache, NVS_ERR_INVALID, "qk_norm_rope_store: null k, v, positions or "
              "cos_sin_cache");
    NVS_CHECK(n_heads == 0 || (q && q_out), NVS_ERR_INVALID, "qk_norm_rope_store: n_heads=%d needs q and q_out",
              n_heads);
    NVS_CHECK(cache_positions > 0, NVS_ERR_INVALID, "qk_norm_rope_store: empty cos_sin_cache");
    NVS_CHECK(slot_mapping == nullptr || (k_cache && v_cache && cache_blocks >= 0 && block_size > 0 &&
                                          cache_block_stride >= 0 && cache_token_stride >= 0 &&
                                          cache_head_stride >= 0),
              NVS_ERR_INVALID, "qk_norm_rope_store: slot_mapping needs k_cache, v_cache and a cache geometry "
              "(blocks >= 0, block_size > 0, strides >= 0)");
    NVS_CHECK(q_token_stride >= static_cast<int64_t>(n_heads) * head_dim &&
                  k_token_stride >= static_cast<int64_t>(n_kv_heads) * head_dim &&
                  v_token_stride >= static_cast<int64_t>(n_kv_heads) * head_dim &&
                  (q_out == nullptr || q_out_token_stride >= static_cast<int64_t>(n_heads) * head_dim) &&
                  (k_out == nullptr || k_out_token_stride >= static_cast<int64_t>(n_kv_heads) * head_dim),
              NVS_ERR_INVALID, "qk_norm_rope_store: a token stride is shorter than its heads x head_dim");
    NVS_CHECK(n_tokens <= 0x7fffffff, NVS_ERR_UNSUPPORTED, "qk_norm_rope_store: too many tokens");
    const int rows = n_heads + 2 * n_kv_heads;
    const int row_blocks = (rows + kRowsPerBlock - 1) / kRowsPerBlock;
    NVS_CHECK(row_blocks <= 65535, NVS_ERR_UNSUPPORTED, "qk_norm_rope_store: too many heads");

    NormRopeArgs a;
    a.q = static_cast<const uint16_t*>(q);
    a.q_ts = q_token_stride;
    a.k = static_cast<const uint16_t*>(k);
    a.k_ts = k_token_stride;
    a.v = static_cast<const uint16_t*>(v);
    a.v_ts = v_token_stride;
    a.pos = positions;
    a.qw = static_cast<const uint16_t*>(q_norm_weight);
    a.kw = static_cast<const uint16_t*>(k_norm_weight);
    a.eps = eps;
    a.cs = cos_sin_cache;
    a.n_cs = cache_positions;
    a.slots = slot_mapping;
    a.geo = nvs::CacheGeometry{slot_mapping != nullptr ? cache_blocks : 0, block_size > 0 ? block_size : 1,
                               cache_block_stride, cache_token_stride, cache_head_stride};
    a.kc = static_cast<uint16_t*>(k_cache);
    a.vc = static_cast<uint16_t*>(v_cache);
    a.qo = static_cast<uint16_t*>(q_out);
    a.qo_ts = q_out_token_stride;
    a.ko = static_cast<uint16_t*>(k_out);
    a.ko_ts = k_out_token_stride;
    a.hq = n_heads;
    a.hkv = n_kv_heads;
    const dim3 grid(static_cast<unsigned>(n_tokens), static_cast<unsigned>(row_blocks));
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (dtype == NVS_DTYPE_BF16) {
        hipLaunchKernelGGL(qk_norm_rope_store_kernel<NVS_DTYPE_BF16>, grid, dim3(64 * kRowsPerBlock), 0, s, a);
    } else {
        hipLaunchKernelGGL(qk_norm_rope_store_kernel<NVS_DTYPE_F16>, grid, dim3(64 * kRowsPerBlock), 0, s, a);
    }
    return nvs::check_launch("qk_norm_rope_store");
}
