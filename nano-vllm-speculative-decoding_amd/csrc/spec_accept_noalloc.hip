// The fused accept without a caller workspace: nvs_spec_accept_noalloc.
// No counterpart in the reference. It serves callers that cannot allocate device memory (code under HIP graph
// capture, serving loops or harnesses that forbid allocation): the accept's per-position records, the dense races'
// state and the per-row counters live in `scratch`, a fixed array of this library in each device's global memory,
// instead of a workspace and a counter buffer handed in. The caller still passes every input and output.
//
// Limits: at most kNoAllocMaxRows batch rows, and records + dense-race state of at most kNoAllocWorkBytes (one
// 32-byte record per verify position: up to 32,768 positions when some row truncates). Larger calls return
// NVS_ERR_UNSUPPORTED before any launch. The array stays allocated on every device the library runs on until the
// process ends. Every call on a device shares that device's array, and calls that overlap on one device (two
// streams, or two host threads) race on it; calls ordered on one stream do not.
#include "nvs_common.hpp"
#include "spec_accept.hpp"

#include <mutex>

namespace {
constexpr int64_t kNoAllocMaxRows = 1024;
constexpr size_t kNoAllocCounterBytes = kNoAllocMaxRows * sizeof(int32_t);   // per-row counters, at the front
constexpr size_t kNoAllocWorkBytes = size_t{1} << 20;                         // records and dense-race state
constexpr int kMaxDevices = 64;
}  // namespace

// In host code `scratch` names a host-side stand-in, not the device array: its device address is resolved per
// device by scratch_address() and only that address is handed to kernels.
static __device__ __align__(256) unsigned char scratch[kNoAllocCounterBytes + kNoAllocWorkBytes];

namespace {

std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of the current device's copy of `scratch`, resolved on the first call on that device (with the
// device current) and kept.
int scratch_address(void** out) {
    int dev = -1;
    hipError_t err = hipGetDevice(&dev);
    NVS_CHECK(err == hipSuccess, NVS_ERR_HIP, "spec_accept_noalloc: hipGetDevice failed: %s", hipGetErrorString(err));
    NVS_CHECK(dev >= 0 && dev < kMaxDevices, NVS_ERR_UNSUPPORTED, "spec_accept_noalloc: device %d above %d", dev,
              kMaxDevices - 1);
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (g_scratch_ptr[dev] == nullptr) {
        void* ptr = nullptr;
        err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        NVS_CHECK(err == hipSuccess && ptr != nullptr, NVS_ERR_HIP,
                  "spec_accept_noalloc: hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                  hipGetErrorString(err));
        g_scratch_ptr[dev] = ptr;
    }
    *out = g_scratch_ptr[dev];
    return NVS_OK;
}

// The row counters must be zero when the accept starts. Every accept leaves them zero, but a call that was never
// completed (or one racing with another) could leave some set, so each call clears its rows first, with a kernel:
// a fill node is safe under graph capture where a memset node is not.
__global__ void clear_counters_kernel(int32_t* counters, int64_t n) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n) counters[i] = 0;
}

}  // namespace

extern "C" int nvs_spec_accept_noalloc(const void* logits, int logits_dtype, int64_t logits_row_stride,
                                       const float* temperatures, const int64_t* top_k, const float* top_p,
                                       int max_top_k, int has_top_p, const float* q, const int64_t* drafts,
                                       const int64_t* verified_lens, const float* uniforms, const float* noise,
                                       int64_t batch, int num_drafts, int64_t n_pos, int64_t vocab,
                                       int64_t* n_accept, int64_t* tail, void* stream) {
    nvs::clear_error();
    NVS_CHECK(batch >= 0 && n_pos >= 0 && vocab > 0 && max_top_k >= 0, NVS_ERR_INVALID,
              "spec_accept_noalloc: bad sizes (batch %lld, n_pos %lld, vocab %lld, max_top_k %d)", (long long)batch,
              (long long)n_pos, (long long)vocab, max_top_k);
    NVS_CHECK(batch <= kNoAllocMaxRows, NVS_ERR_UNSUPPORTED,
              "spec_accept_noalloc: batch %lld above the scratch's %lld rows", (long long)batch,
              (long long)kNoAllocMaxRows);
    const size_t need = nvs::spec_accept_workspace_bytes(batch, n_pos, vocab, max_top_k);
    NVS_CHECK(need <= kNoAllocWorkBytes, NVS_ERR_UNSUPPORTED,
              "spec_accept_noalloc: %zu bytes of records needed (n_pos %lld, vocab %lld), the scratch holds %zu",
              need, (long long)n_pos, (long long)vocab, kNoAllocWorkBytes);
    if (batch == 0) return NVS_OK;
    void* base = nullptr;
    const int st = scratch_address(&base);
    if (st != NVS_OK) return st;
    int32_t* counters = static_cast<int32_t*>(base);
    void* work = static_cast<unsigned char*>(base) + kNoAllocCounterBytes;
    hipStream_t s = static_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(clear_counters_kernel, dim3(static_cast<unsigned>((batch + 255) / 256)), dim3(256), 0, s,
                       counters, batch);
    const int lst = nvs::check_launch("spec_accept_noalloc counter clear");
    if (lst != NVS_OK) return lst;
    return nvs::spec_accept_dense_q(logits, logits_dtype, logits_row_stride, temperatures, top_k, top_p, max_top_k,
                                    has_top_p, q, drafts, verified_lens, uniforms, noise, batch, num_drafts, n_pos,
                                    vocab, n_accept, tail, counters, work, kNoAllocWorkBytes, stream);
}
