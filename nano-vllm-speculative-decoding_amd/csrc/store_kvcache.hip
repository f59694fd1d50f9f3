// Paged KV store: writes each new token's K and V rows into its cache slot.
// Reference: store_kvcache_kernel / store_kvcache, nanovllm/layers/attention.py:10-40.
//
// The op is a byte copy (bit-exact for every dtype). One wavefront copies one token row of K and V; a 256-thread
// workgroup covers 4 tokens. When every pointer and row stride is 16-byte aligned each lane moves 16 B per access
// (a full 2 KB bf16 row of 8 kv heads x 128 dims is 2 accesses per lane per tensor); otherwise 2-byte units.
// The cache may be token-major or head-major (any block / token / head strides, see nvs::CacheGeometry).
#include "nvs_common.hpp"

namespace {

constexpr int kTokensPerBlock = 4;
constexpr int kThreads = 64 * kTokensPerBlock;

// geo's strides are in Units; head h of a token row is head_units Units at row offset h * head_units.
template <typename Unit>
__global__ __launch_bounds__(kThreads) void store_kvcache_kernel(
    const Unit* __restrict__ key, int64_t key_stride_units,
    const Unit* __restrict__ value, int64_t value_stride_units,
    Unit* __restrict__ k_cache, Unit* __restrict__ v_cache, nvs::CacheGeometry geo,
    const int32_t* __restrict__ slot_mapping, int64_t n_tokens, int n_heads, int head_units) {
    const int64_t token = static_cast<int64_t>(blockIdx.x) * kTokensPerBlock + (threadIdx.x >> 6);
    if (token >= n_tokens) return;
    const int64_t slot = slot_mapping[token];
    if (slot < 0 || slot >= geo.slots()) return;  // -1 marks a padding token (batch_metadata.py:10)
    const int lane = threadIdx.x & 63;
    const Unit* ksrc = key + token * key_stride_units;
    const Unit* vsrc = value + token * value_stride_units;
    const int64_t base = geo.offset(slot, 0);
    const int row_units = n_heads * head_units;
    for (int u = lane; u < row_units; u += 64) {
        const int h = u / head_units;
        const int64_t dst = base + h * geo.head_stride + (u - h * head_units);
        const Unit kv = ksrc[u];
        const Unit vv = vsrc[u];
        k_cache[dst] = kv;
        v_cache[dst] = vv;
    }
}

template <typename Unit>
int launch(const void* key, int64_t key_row_stride, const void* value, int64_t value_row_stride, void* k_cache,
           void* v_cache, nvs::CacheGeometry geo, const int32_t* slot_mapping, int64_t n_tokens, int n_kv_heads,
           int head_dim, int es, hipStream_t s) {
    const int64_t per = static_cast<int64_t>(sizeof(Unit)) / es;  // elements per Unit
    geo.block_stride /= per;
    geo.token_stride /= per;
    geo.head_stride /= per;
    const dim3 grid(static_cast<unsigned>((n_tokens + kTokensPerBlock - 1) / kTokensPerBlock));
    hipLaunchKernelGGL(store_kvcache_kernel<Unit>, grid, dim3(kThreads), 0, s, static_cast<const Unit*>(key),
                       key_row_stride / per, static_cast<const Unit*>(value), value_row_stride / per,
                       static_cast<Unit*>(k_cache), static_cast<Unit*>(v_cache), geo, slot_mapping, n_tokens,
                       n_kv_heads, static_cast<int>(head_dim / per));
    return nvs::check_launch("store_kvcache");
}

}  // namespace

extern "C" int nvs_store_kvcache(const void* key, int64_t key_row_stride, const void* value,
                                 int64_t value_row_stride, void* k_cache, void* v_cache, int64_t cache_blocks,
                                 int64_t block_size, int64_t cache_block_stride, int64_t cache_token_stride,
                                 int64_t cache_head_stride, const int32_t* slot_mapping, int64_t n_tokens,
                                 int n_kv_heads, int head_dim, int dtype, void* stream) {
    nvs::clear_error();
    const int es = nvs::dtype_size(dtype);
    NVS_CHECK(es > 0, NVS_ERR_INVALID, "store_kvcache: unknown dtype %d", dtype);
    NVS_CHECK(n_tokens >= 0 && n_kv_heads > 0 && head_dim > 0 && cache_blocks >= 0 && block_size > 0,
              NVS_ERR_INVALID,
              "store_kvcache: bad sizes n_tokens=%lld n_kv_heads=%d head_dim=%d cache_blocks=%lld block_size=%lld",
              (long long)n_tokens, n_kv_heads, head_dim, (long long)cache_blocks, (long long)block_size);
    NVS_CHECK(cache_block_stride >= 0 && cache_token_stride >= 0 && cache_head_stride >= 0, NVS_ERR_INVALID,
              "store_kvcache: negative cache stride");
    if (n_tokens == 0) return NVS_OK;
    NVS_CHECK(key && value && k_cache && v_cache && slot_mapping, NVS_ERR_INVALID,
              "store_kvcache: null pointer");
    const int64_t row = static_cast<int64_t>(n_kv_heads) * head_dim;
    NVS_CHECK(key_row_stride >= row && value_row_stride >= row, NVS_ERR_INVALID,
              "store_kvcache: row strides (%lld, %lld) shorter than a row of %lld elements",
              (long long)key_row_stride, (long long)value_row_stride, (long long)row);
    const nvs::CacheGeometry geo{cache_blocks, block_size, cache_block_stride, cache_token_stride, cache_head_stride};
    auto mult = [es](int64_t elems, int bytes) { return (elems * es) % bytes == 0; };
    const bool strides16 = mult(head_dim, 16) && mult(key_row_stride, 16) && mult(value_row_stride, 16) &&
                           mult(cache_block_stride, 16) && mult(cache_token_stride, 16) &&
                           mult(cache_head_stride, 16);
    const bool vec = strides16 && nvs::aligned16(key) && nvs::aligned16(value) && nvs::aligned16(k_cache) &&
                     nvs::aligned16(v_cache);
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (vec) {
        return launch<uint4>(key, key_row_stride, value, value_row_stride, k_cache, v_cache, geo, slot_mapping,
                             n_tokens, n_kv_heads, head_dim, es, s);
    }
    if (es == 4) {
        return launch<uint32_t>(key, key_row_stride, value, value_row_stride, k_cache, v_cache, geo, slot_mapping,
                                n_tokens, n_kv_heads, head_dim, es, s);
    }
    return launch<uint16_t>(key, key_row_stride, value, value_row_stride, k_cache, v_cache, geo, slot_mapping,
                            n_tokens, n_kv_heads, head_dim, es, s);
}
