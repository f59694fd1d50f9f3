// RMSNorm (with the residual add) and SiLU-and-mul of a Qwen3 decoder layer: the elementwise steps between the
// projections of a verify forward.
// Reference:
//   RMSNorm.rms_forward / add_rms_forward, nanovllm/layers/layernorm.py:15-46
//       x = float(x) [+ float(residual)]; residual = dtype(x); x *= rsqrt(mean(x^2) + eps); out = dtype(x) * weight
//   SiluAndMul.forward, nanovllm/layers/activation.py:8-11
//       gate, up = x.chunk(2, -1); out = silu(gate) * up
//
// RMSNorm: one 256-thread workgroup per row; each thread holds up to 4 pieces of 8 elements (hidden <= 8192,
// a multiple of 8), loaded once with 16-byte loads. The sum of squares is an fp32 sum in a fixed order (per
// thread, then DPP inside each wave, then the 4 waves), so the result does not depend on the launch. The scale is
// a correctly rounded 1 / sqrt(var + eps); the output is rounded to the dtype before the weight product and again
// after it, as the reference's explicit casts do. Writing the output over x is allowed: every thread writes only
// the elements it read itself.
// SiLU-and-mul: one thread per 8 outputs, silu(g) * u computed in fp32 and rounded once (the reference runs under
// torch.compile, which keeps the intermediate in fp32).
#include "nvs_common.hpp"

namespace {

constexpr int kNormThreads = 256;
constexpr int kPiece = 8;          // elements per 16-byte load
constexpr int kMaxPieces = 4;      // per thread: hidden <= 256 * 8 * 4
constexpr int kMaxHidden = kNormThreads * kPiece * kMaxPieces;

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
__device__ __forceinline__ void unpack(const uint4& v, float (&f)[kPiece]) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        f[2 * i] = to_f<DT>(static_cast<uint16_t>(w[i] & 0xffffu));
        f[2 * i + 1] = to_f<DT>(static_cast<uint16_t>(w[i] >> 16));
    }
}

template <int DT>
__device__ __forceinline__ uint4 pack(const float (&f)[kPiece]) {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
        w[i] = static_cast<uint32_t>(to_bits<DT>(f[2 * i])) | (static_cast<uint32_t>(to_bits<DT>(f[2 * i + 1])) << 16);
    return make_uint4(w[0], w[1], w[2], w[3]);
}

struct NormArgs {
    const uint16_t* x;
    int64_t x_rs;
    uint16_t* res;   // null: no residual
    int64_t res_rs;
    const uint16_t* w;
    float eps;
    uint16_t* out;
    int64_t out_rs;
    int hidden;
};

template <int DT>
__global__ __launch_bounds__(kNormThreads) void rms_norm_kernel(NormArgs a) {
#pragma clang fp contract(off)
    __shared__ float wsum[kNormThreads / 64];
    const int64_t row = blockIdx.x;
    const int pieces = a.hidden / kPiece;
    const uint4* xp = reinterpret_cast<const uint4*>(a.x + row * a.x_rs);
    uint4* rp = a.res != nullptr ? reinterpret_cast<uint4*>(a.res + row * a.res_rs) : nullptr;
    float v[kMaxPieces][kPiece];
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < kMaxPieces; ++i) {
        const int p = static_cast<int>(threadIdx.x) + i * kNormThreads;
        if (p < pieces) {
            unpack<DT>(xp[p], v[i]);
            if (rp != nullptr) {
                float r[kPiece];
                unpack<DT>(rp[p], r);
#pragma unroll
                for (int e = 0; e < kPiece; ++e) v[i][e] = v[i][e] + r[e];
                rp[p] = pack<DT>(v[i]);   // the new residual: the sum rounded to the dtype
            }
#pragma unroll
            for (int e = 0; e < kPiece; ++e) ss += v[i][e] * v[i][e];
        }
    }
    ss = nvs::wave_sum(ss);
    if ((threadIdx.x & 63) == 0) wsum[threadIdx.x >> 6] = ss;
    __syncthreads();
    const float total = (wsum[0] + wsum[1]) + (wsum[2] + wsum[3]);
    const float var = total / static_cast<float>(a.hidden);
    const float scale = 1.0f / sqrtf(var + a.eps);
    const uint4* wp = reinterpret_cast<const uint4*>(a.w);
    uint4* op = reinterpret_cast<uint4*>(a.out + row * a.out_rs);
#pragma unroll
    for (int i = 0; i < kMaxPieces; ++i) {
        const int p = static_cast<int>(threadIdx.x) + i * kNormThreads;
        if (p < pieces) {
            float w[kPiece];
            unpack<DT>(wp[p], w);
            float o[kPiece];
#pragma unroll
            for (int e = 0; e < kPiece; ++e) o[e] = to_f<DT>(to_bits<DT>(v[i][e] * scale)) * w[e];
            op[p] = pack<DT>(o);
        }
    }
}

struct SiluArgs {
    const uint16_t* x;
    int64_t x_rs;
    uint16_t* out;
    int64_t out_rs;
    int width;         // outputs per row; the row holds the gate [0, width) then the up part [width, 2 width)
    int64_t pieces;    // n_rows * width / 8
};

template <int DT>
__global__ __launch_bounds__(256) void silu_mul_kernel(SiluArgs a) {
#pragma clang fp contract(off)
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= a.pieces) return;
    const int per_row = a.width / kPiece;
    const int64_t row = i / per_row;
    const int col = static_cast<int>(i - row * per_row) * kPiece;
    const uint16_t* src = a.x + row * a.x_rs + col;
    float g[kPiece], u[kPiece], o[kPiece];
    unpack<DT>(*reinterpret_cast<const uint4*>(src), g);
    unpack<DT>(*reinterpret_cast<const uint4*>(src + a.width), u);
#pragma unroll
    for (int e = 0; e < kPiece; ++e) o[e] = g[e] / (1.0f + expf(-g[e])) * u[e];
    *reinterpret_cast<uint4*>(a.out + row * a.out_rs + col) = pack<DT>(o);
}

bool aligned_rows(const void* p, int64_t row_stride) { return nvs::aligned16(p) && row_stride % kPiece == 0; }

}  // namespace

extern "C" int nvs_rms_norm(const void* x, int64_t x_row_stride, void* residual, int64_t residual_row_stride,
                            const void* weight, float eps, void* out, int64_t out_row_stride, int64_t n_rows,
                            int hidden, int dtype, void* stream) {
    nvs::clear_error();
    NVS_CHECK(dtype == NVS_DTYPE_BF16 || dtype == NVS_DTYPE_F16, NVS_ERR_UNSUPPORTED,
              "rms_norm: dtype %d unsupported (bf16 or fp16)", dtype);
    NVS_CHECK(n_rows >= 0 && hidden > 0, NVS_ERR_INVALID, "rms_norm: bad sizes n_rows=%lld hidden=%d",
              (long long)n_rows, hidden);
    NVS_CHECK(hidden % kPiece == 0 && hidden <= kMaxHidden, NVS_ERR_UNSUPPORTED,
              "rms_norm: hidden %d unsupported (a multiple of 8, at most %d)", hidden, kMaxHidden);
    if (n_rows == 0) return NVS_OK;
    NVS_CHECK(x && weight && out, NVS_ERR_INVALID, "rms_norm: null x, weight or out");
    NVS_CHECK(n_rows <= 0x7fffffff, NVS_ERR_UNSUPPORTED, "rms_norm: too many rows");
    NVS_CHECK(x_row_stride >= hidden && out_row_stride >= hidden &&
                  (residual == nullptr || residual_row_stride >= hidden),
              NVS_ERR_INVALID, "rms_norm: a row stride is shorter than hidden");
    NVS_CHECK(aligned_rows(x, x_row_stride) && aligned_rows(out, out_row_stride) && nvs::aligned16(weight) &&
                  (residual == nullptr || aligned_rows(residual, residual_row_stride)),
              NVS_ERR_UNSUPPORTED, "rms_norm: pointers must be 16-byte aligned and row strides multiples of 8");
    NormArgs a;
    a.x = static_cast<const uint16_t*>(x);
    a.x_rs = x_row_stride;
    a.res = static_cast<uint16_t*>(residual);
    a.res_rs = residual_row_stride;
    a.w = static_cast<const uint16_t*>(weight);
    a.eps = eps;
    a.out = static_cast<uint16_t*>(out);
    a.out_rs = out_row_stride;
    a.hidden = hidden;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const dim3 grid(static_cast<unsigned>(n_rows));
    if (dtype == NVS_DTYPE_BF16) {
        hipLaunchKernelGGL(rms_norm_kernel<NVS_DTYPE_BF16>, grid, dim3(kNormThreads), 0, s, a);
    } else {
        hipLaunchKernelGGL(rms_norm_kernel<NVS_DTYPE_F16>, grid, dim3(kNormThreads), 0, s, a);
    }
    return nvs::check_launch("rms_norm");
}

extern "C" int nvs_silu_and_mul(const void* x, int64_t x_row_stride, void* out, int64_t out_row_stride,
                                int64_t n_rows, int width, int dtype, void* stream) {
    nvs::clear_error();
    NVS_CHECK(dtype == NVS_DTYPE_BF16 || dtype == NVS_DTYPE_F16, NVS_ERR_UNSUPPORTED,
              "silu_and_mul: dtype %d unsupported (bf16 or fp16)", dtype);
    NVS_CHECK(n_rows >= 0 && width > 0, NVS_ERR_INVALID, "silu_and_mul: bad sizes n_rows=%lld width=%d",
              (long long)n_rows, width);
    NVS_CHECK(width % kPiece == 0, NVS_ERR_UNSUPPORTED, "silu_and_mul: width %d is not a multiple of 8", width);
    if (n_rows == 0) return NVS_OK;
    NVS_CHECK(x && out, NVS_ERR_INVALID, "silu_and_mul: null x or out");
    NVS_CHECK(x_row_stride >= 2 * static_cast<int64_t>(width) && out_row_stride >= width, NVS_ERR_INVALID,
              "silu_and_mul: a row stride is shorter than the row");
    NVS_CHECK(aligned_rows(x, x_row_stride) && aligned_rows(out, out_row_stride), NVS_ERR_UNSUPPORTED,
              "silu_and_mul: pointers must be 16-byte aligned and row strides multiples of 8");
    SiluArgs a;
    a.x = static_cast<const uint16_t*>(x);
    a.x_rs = x_row_stride;
    a.out = static_cast<uint16_t*>(out);
    a.out_rs = out_row_stride;
    a.width = width;
    a.pieces = n_rows * (width / kPiece);
    const int64_t blocks = (a.pieces + 255) / 256;
    NVS_CHECK(blocks <= 0x7fffffff, NVS_ERR_UNSUPPORTED, "silu_and_mul: too large");
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (dtype == NVS_DTYPE_BF16) {
        hipLaunchKernelGGL(silu_mul_kernel<NVS_DTYPE_BF16>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s, a);
    } else {
        hipLaunchKernelGGL(silu_mul_kernel<NVS_DTYPE_F16>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s, a);
    }
    return nvs::check_launch("silu_and_mul");
}
