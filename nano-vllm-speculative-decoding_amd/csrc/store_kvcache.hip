// Paged KV store: writes each new token's K and V rows into its cache slot.
// Reference: store_kvcache_kernel / store_kvcache, nanovllm/layers/attention.py:10-40.
//
// The op is a byte copy (bit-exact for every dtype). One wavefront copies one token row of K and V; a 256-thread
// workgroup covers 4 tokens. When every pointer and row stride is 16-byte aligned each lane moves 16 B per access
// (a full 2 KB bf16 row of 8 kv heads x 128 dims is 2 accesses per lane per tensor); otherwise 2-byte units.
#include "nvs_common.hpp"

namespace {

constexpr int kTokensPerBlock = 4;
constexpr int kThreads = 64 * kTokensPerBlock;

template <typename Unit>
__global__ __launch_bounds__(kThreads) void store_kvcache_kernel(
    const Unit* __restrict__ key, int64_t key_stride_units,
    const Unit* __restrict__ value, int64_t value_stride_units,
    Unit* __restrict__ k_cache, Unit* __restrict__ v_cache, int64_t cache_slots,
    const int32_t* __restrict__ slot_mapping, int64_t n_tokens, int row_units) {
    const int64_t token = static_cast<int64_t>(blockIdx.x) * kTokensPerBlock + (threadIdx.x >> 6);
    if (token >= n_tokens) return;
    const int64_t slot = slot_mapping[token];
    if (slot < 0 || slot >= cache_slots) return;  // -1 marks a padding token (batch_metadata.py:10)
    const int lane = threadIdx.x & 63;
    const Unit* ksrc = key + token * key_stride_units;
    const Unit* vsrc = value + token * value_stride_units;
    Unit* kdst = k_cache + slot * row_units;
    Unit* vdst = v_cache + slot * row_units;
    for (int u = lane; u < row_units; u += 64) {
        const Unit kv = ksrc[u];
        const Unit vv = vsrc[u];
        kdst[u] = kv;
        vdst[u] = vv;
    }
}

}  // namespace

extern "C" int nvs_store_kvcache(const void* key, int64_t key_row_stride, const void* value,
                                 int64_t value_row_stride, void* k_cache, void* v_cache, int64_t cache_slots,
                                 const int32_t* slot_mapping, int64_t n_tokens, int n_kv_heads, int head_dim,
                                 int dtype, void* stream) {
    nvs::clear_error();
    const int es = nvs::dtype_size(dtype);
    NVS_CHECK(es > 0, NVS_ERR_INVALID, "store_kvcache: unknown dtype %d", dtype);
    NVS_CHECK(n_tokens >= 0 && n_kv_heads > 0 && head_dim > 0 && cache_slots >= 0, NVS_ERR_INVALID,
              "store_kvcache: bad sizes n_tokens=%lld n_kv_heads=%d head_dim=%d cache_slots=%lld",
              (long long)n_tokens, n_kv_heads, head_dim, (long long)cache_slots);
    if (n_tokens == 0) return NVS_OK;
    NVS_CHECK(key && value && k_cache && v_cache && slot_mapping, NVS_ERR_INVALID,
              "store_kvcache: null pointer");
    const int64_t row = static_cast<int64_t>(n_kv_heads) * head_dim;
    NVS_CHECK(key_row_stride >= row && value_row_stride >= row, NVS_ERR_INVALID,
              "store_kvcache: row strides (%lld, %lld) shorter than a row of %lld elements",
              (long long)key_row_stride, (long long)value_row_stride, (long long)row);
    const int64_t row_bytes = row * es;
    const bool vec = nvs::aligned16(key) && nvs::aligned16(value) && nvs::aligned16(k_cache) &&
                     nvs::aligned16(v_cache) && (row_bytes % 16 == 0) && ((key_row_stride * es) % 16 == 0) &&
                     ((value_row_stride * es) % 16 == 0);
    const dim3 grid(static_cast<unsigned>((n_tokens + kTokensPerBlock - 1) / kTokensPerBlock));
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (vec) {
        const int64_t per = 16 / es;  // elements per 16-byte unit
        hipLaunchKernelGGL(store_kvcache_kernel<uint4>, grid, dim3(kThreads), 0, s,
                           static_cast<const uint4*>(key), key_row_stride / per,
                           static_cast<const uint4*>(value), value_row_stride / per,
                           static_cast<uint4*>(k_cache), static_cast<uint4*>(v_cache), cache_slots, slot_mapping,
                           n_tokens, static_cast<int>(row_bytes / 16));
    } else if (es == 4) {
        hipLaunchKernelGGL(store_kvcache_kernel<uint32_t>, grid, dim3(kThreads), 0, s,
                           static_cast<const uint32_t*>(key), key_row_stride,
                           static_cast<const uint32_t*>(value), value_row_stride,
                           static_cast<uint32_t*>(k_cache), static_cast<uint32_t*>(v_cache), cache_slots,
                           slot_mapping, n_tokens, static_cast<int>(row));
    } else {
        hipLaunchKernelGGL(store_kvcache_kernel<uint16_t>, grid, dim3(kThreads), 0, s,
                           static_cast<const uint16_t*>(key), key_row_stride,
                           static_cast<const uint16_t*>(value), value_row_stride,
                           static_cast<uint16_t*>(k_cache), static_cast<uint16_t*>(v_cache), cache_slots,
                           slot_mapping, n_tokens, static_cast<int>(row));
    }
    return nvs::check_launch("store_kvcache");
}
