// Shared helpers of the gfx950 kernels: status/error plumbing, dtype loads, launch checks.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_bf16.h>
#include <hip/hip_fp16.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <string>

#include "nvs_amd.h"  // include/ is on the include path (build.py)

namespace nvs {

// Thread-local message of the last failed call, returned by nvs_last_error().
void set_error(const char* fmt, ...);
void clear_error();

#define NVS_CHECK(cond, status, ...)          \
    do {                                      \
        if (!(cond)) {                        \
            ::nvs::set_error(__VA_ARGS__);    \
            return (status);                  \
        }                                     \
    } while (0)

// After a kernel launch: turn a runtime launch error into NVS_ERR_HIP.
int check_launch(const char* what);

__host__ __device__ inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

inline size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

__host__ __device__ inline int dtype_size(int dtype) {
    switch (dtype) {
        case NVS_DTYPE_F32: return 4;
        case NVS_DTYPE_BF16: return 2;
        case NVS_DTYPE_F16: return 2;
        default: return 0;
    }
}

// A paged K/V cache seen as [blocks, block_size, kv heads, head_dim] with element strides for the first three
// dimensions (the head dimension is contiguous). Slot s is token s % block_size of block s / block_size. The
// token-major layout [blocks, block_size, Hkv, D] has strides (block_size*Hkv*D, Hkv*D, D); the head-major layout
// [blocks, Hkv, block_size, D], where every (block, head) is one contiguous run, has (Hkv*block_size*D, D,
// block_size*D).
struct CacheGeometry {
    int64_t blocks;
    int64_t block_size;
    int64_t block_stride, token_stride, head_stride;
    __host__ __device__ int64_t slots() const { return blocks * block_size; }
    __host__ __device__ int64_t offset(int64_t slot, int head) const {
        const int64_t b = slot / block_size;
        return b * block_stride + (slot - b * block_size) * token_stride + head * head_stride;
    }
};

// ---------------------------------------------------------------- device helpers

// bf16 / f16 bit patterns -> fp32 (exact).
__device__ __forceinline__ float bf16_bits_to_float(uint16_t b) {
    return __uint_as_float(static_cast<uint32_t>(b) << 16);
}

__device__ __forceinline__ float f16_bits_to_float(uint16_t b) {
    return __half2float(__ushort_as_half(b));
}

// fp32 -> bf16 bits, round to nearest even (NaN kept quiet).
__device__ __forceinline__ uint16_t float_to_bf16_bits(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return static_cast<uint16_t>(u >> 16);
}

template <int DT>
__device__ __forceinline__ float load_as_float(const void* base, int64_t idx) {
    if constexpr (DT == NVS_DTYPE_F32) {
        return static_cast<const float*>(base)[idx];
    } else if constexpr (DT == NVS_DTYPE_BF16) {
        return bf16_bits_to_float(static_cast<const uint16_t*>(base)[idx]);
    } else {
        return f16_bits_to_float(static_cast<const uint16_t*>(base)[idx]);
    }
}

// Wave reductions through DPP (no LDS round trips): rotations by 8, 4, 2 and 1 inside each 16-lane row leave
// every lane with its row's result; row_bcast:15 folds row 0 into row 1 and row 2 into row 3, row_bcast:31 folds
// rows 0-1 into rows 2-3, so lane 63 holds the wave's result, which readlane hands to every lane. Lanes of rows
// a broadcast does not write get `old`: the identity for a sum, the lane's own value for a max. The whole wave
// must be active.
template <int CTRL, int ROWS>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t old, uint32_t src) {
    return static_cast<uint32_t>(
        __builtin_amdgcn_update_dpp(static_cast<int>(old), static_cast<int>(src), CTRL, ROWS, 0xf, false));
}

// fp32 sum over the wave in a fixed order (the same result on every lane).
__device__ __forceinline__ float wave_sum(float v) {
    v += __uint_as_float(dpp_u32<0x128, 0xf>(0u, __float_as_uint(v)));   // row_ror:8
    v += __uint_as_float(dpp_u32<0x124, 0xf>(0u, __float_as_uint(v)));   // row_ror:4
    v += __uint_as_float(dpp_u32<0x122, 0xf>(0u, __float_as_uint(v)));   // row_ror:2
    v += __uint_as_float(dpp_u32<0x121, 0xf>(0u, __float_as_uint(v)));   // row_ror:1
    v += __uint_as_float(dpp_u32<0x142, 0xa>(0u, __float_as_uint(v)));   // row_bcast:15
    v += __uint_as_float(dpp_u32<0x143, 0xc>(0u, __float_as_uint(v)));   // row_bcast:31
    return __uint_as_float(static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(__float_as_uint(v)), 63)));
}

// Order-preserving map of fp32 onto uint32: a < b  <=>  key(a) < key(b) (for non-NaN; -0 < +0).
__device__ __forceinline__ uint32_t float_key(float f) {
    uint32_t u = __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float key_float(uint32_t k) {
    uint32_t u = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
    return __uint_as_float(u);
}

}  // namespace nvs
