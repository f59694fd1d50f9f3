// Speculative sampler for gfx950: truncation -> softmax -> rejection test -> residual / bonus race.
// Reference: nanovllm/layers/spec_sampler.py (probs_from_logits :65-69, truncate_logits :72-96, race / sample
// :99-111, accept_random(_varlen) :114-150, accept_greedy(_varlen) :153-169, _verified_positions :172-180) as
// dispatched by SpeculativeDecoder._accept, nanovllm/engine/speculative.py:450-462.
//
// Selection kernel (one 512-thread workgroup per logit row = verify position):
//   * one coalesced pass over the row: s = logit / temperature (IEEE division, skipped when it is exactly 1);
//   * rows that truncate (top_k > 0): every element at or above a running lower bound tau of the row's
//     max_top_k-th largest value is appended to a lane-private candidate list in LDS. tau starts from the first
//     8192 elements: each wave takes the ceil(K/8)-th largest of its 64 lane maxima, tau is the smallest of the 8,
//     so at least K elements lie at or above it. A wave whose lane fills 12 of its 16 slots raises its bound from a
//     histogram of its lists and drops what falls below it. The lists therefore hold every element >= the K-th
//     largest, ties included, and nothing else is needed;
//   * a 256-bin histogram of the listed keys and a count inside the bin holding the rank-th largest give the
//     threshold (rank = min(top_k, K)); top-p sorts the candidates above it and runs the nucleus softmax / cumsum of
//     truncate_logits; the kept set is {s >= threshold} (ties kept);
//   * rows that do not truncate (top_k = 0) keep an online max / sum-exp instead;
//   * a lane whose list overflows (thousands of tied values, adversarial order) sends the row to an exact radix
//     select over the row itself; windows wider than the lists (max_top_k > 1024) take that path by design.
// Then, depending on the entry point: write dense probabilities (probs_from_logits), write truncated logits
// (truncate_logits), or (fused accept) evaluate this position's accept test u * q[d] < p[d] and its race:
// argmax over the kept set of w / E with w = p (bonus position) or max(p - q, 0) (first rejection here), reading
// q and E only at the kept indices. The batch row's last position to finish (counted on a per-row counter) counts
// the accepted prefix and picks the race of the position that follows it; rows that do not truncate race over the
// whole vocabulary in a second launch.
#include "nvs_common.hpp"
#include "spec_accept.hpp"

#include <cmath>
#include <type_traits>

namespace {

constexpr int kSelThreads = 512;
constexpr int kSelWaves = kSelThreads / 64;
constexpr int kVpt = 16;                       // values per thread per batch
constexpr int kBatch = kSelThreads * kVpt;     // 8192 elements per batch
constexpr int kLaneCap = 16;                   // candidate slots per lane during the streaming pass
constexpr int kWaveSlots = kLaneCap * 64;      // a wave's slots: slot s of lane l at s * 64 + l
constexpr int kCap = kSelWaves * kWaveSlots;   // LDS candidate capacity (8192)
constexpr int kMaxTopK = 1024;
constexpr int kRaceChunk = 8192;               // vocabulary chunk of the dense race kernels (256 threads)
constexpr int kRacePer = kRaceChunk / 4 / 256;  // 16-byte pieces per thread and array

enum Mode { kModeAccept = 0, kModeProbs = 1, kModeTruncate = 2, kModeMarkov = 3 };

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kFlagDense = 1;  // the race of this position must scan the whole vocabulary

struct PosRecord {
    float m;        // max of the kept set
    float z;        // sum of exp(s - m) over the kept set
    float theta;    // truncation threshold (-inf when nothing is truncated)
    float temp;     // temperature of the row
    int flags;
    int acc;        // accept decision of the draft verified at this position
    int64_t race;   // winner of this position's race (valid unless kFlagDense)
};
static_assert(sizeof(PosRecord) == 32, "record layout");

// The race of a batch row whose tail position does not truncate, handed by the accept kernel's row finish to
// dense_race_chunk_kernel (used when no row truncates, so the host launches it after the accept kernel).
struct DenseRace {
    int64_t pos;     // logit row of the position after the accepted prefix
    int64_t qrow;    // q row b * k + min(n, k - 1); -1 for the bonus position (w = p)
    float m, z, temp;
    int valid;       // 1: this row's tail comes from the dense race
};

// Records cross workgroups (and XCDs) through device-scope atomic stores and loads, which the gfx950 backend
// performs at the device's coherence point (sc1) rather than in an XCD's own L2. That keeps them out of the L2
// write-back a release fence would force on every position.
__device__ __forceinline__ void store_record(PosRecord* dst, const PosRecord& r) {
    uint64_t w[4];
    __builtin_memcpy(w, &r, sizeof(w));
    uint64_t* d = reinterpret_cast<uint64_t*>(dst);
#pragma unroll
    for (int i = 0; i < 4; ++i) __hip_atomic_store(d + i, w[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ PosRecord load_record(const PosRecord* src) {
    uint64_t w[4];
    const uint64_t* s = reinterpret_cast<const uint64_t*>(src);
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = __hip_atomic_load(s + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    PosRecord r;
    __builtin_memcpy(&r, w, sizeof(w));
    return r;
}

struct SelArgs {
    const void* logits;
    int64_t row_stride;
    int64_t n_pos;
    int64_t vocab;
    const float* temps;
    const int64_t* top_k;
    const float* top_p;
    int max_top_k;
    int has_top_p;
    int64_t pos_per_param;
    // fused accept
    const float* q;          // dense q [batch, k, vocab], or null with candidate rows below
    const int32_t* q_ids;    // candidate rows of q: [batch * k, q_stride] token ids (-1: none) ...
    const float* q_probs;    // ... and their probabilities
    int q_cand;
    int64_t q_stride;
    const int64_t* drafts;
    const int64_t* lens;
    const float* uniforms;
    const float* noise;
    int64_t batch;
    int k;
    PosRecord* rec;
    int* counters;        // [batch] finished positions per row; zero between calls
    DenseRace* dense_race;   // non-null: rows without truncation leave their race to the dense race kernels
    uint64_t* dense_partial; // [batch, dense_chunks] best keys of the dense race's chunks
    int dense_chunks;
    int64_t* n_accept;
    int64_t* tail;
    // dense outputs
    float* out;
    int64_t out_stride;
    // Markov draw: candidates per position, noise by candidate rank, sparse outputs and the drawn token
    int n_cand;
    int64_t noise_stride;
    int32_t* cand_ids;
    float* cand_probs;
    int64_t cand_stride;
    int64_t* draws;
    int64_t draws_stride;
};

// ---------------------------------------------------------------- wave / workgroup helpers

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }

// Compiler-only memory fence (keeps LDS accesses of one wave in program order for the compiler; the hardware
// already executes them in order).
__device__ __forceinline__ void compiler_fence_s() { asm volatile("" ::: "memory"); }

// Wave reductions through DPP (nvs::dpp_u32): the max forms use the lane's own value as `old`.
using nvs::dpp_u32;
using nvs::wave_sum;

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
    v = max(v, dpp_u32<0x128, 0xf>(v, v));
    v = max(v, dpp_u32<0x124, 0xf>(v, v));
    v = max(v, dpp_u32<0x122, 0xf>(v, v));
    v = max(v, dpp_u32<0x121, 0xf>(v, v));
    v = max(v, dpp_u32<0x142, 0xa>(v, v));
    v = max(v, dpp_u32<0x143, 0xc>(v, v));
    return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), 63));
}

template <int CTRL, int ROWS>
__device__ __forceinline__ uint64_t dpp_max_u64(uint64_t v) {
    const uint32_t lo = static_cast<uint32_t>(v), hi = static_cast<uint32_t>(v >> 32);
    const uint64_t o = (static_cast<uint64_t>(dpp_u32<CTRL, ROWS>(hi, hi)) << 32) | dpp_u32<CTRL, ROWS>(lo, lo);
    return v > o ? v : o;
}

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
    v = dpp_max_u64<0x128, 0xf>(v);
    v = dpp_max_u64<0x124, 0xf>(v);
    v = dpp_max_u64<0x122, 0xf>(v);
    v = dpp_max_u64<0x121, 0xf>(v);
    v = dpp_max_u64<0x142, 0xa>(v);
    v = dpp_max_u64<0x143, 0xc>(v);
    const int lo = __builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(v)), 63);
    const int hi = __builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(v >> 32)), 63);
    return (static_cast<uint64_t>(static_cast<uint32_t>(hi)) << 32) | static_cast<uint32_t>(lo);
}

// Inclusive prefix sum over the wave.
__device__ __forceinline__ double wave_scan_incl_f64(double v) {
    const int l = lane_id();
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const double w = __shfl_up(v, o);
        if (l >= o) v += w;
    }
    return v;
}

__device__ __forceinline__ int64_t wave_scan_incl_i64(int64_t v) {
    const int l = lane_id();
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int64_t w = __shfl_up(v, o);
        if (l >= o) v += w;
    }
    return v;
}

// Inclusive prefix sum of one integer per lane over the wave through DPP (no LDS round trips): Hillis-Steele
// shifts by 1, 2, 4 and 8 inside each 16-lane row, then row 0's total into row 1 and row 2's into row 3
// (row_bcast:15), then rows 0-1's total into rows 2 and 3 (row_bcast:31). Masked rows and lanes shifted in
// from outside a row add 0.
__device__ __forceinline__ int wave_scan_incl_dpp(int x) {
    x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xf, 0xf, true);   // row_shr:1
    x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xf, 0xf, true);   // row_shr:2
    x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xf, 0xf, true);   // row_shr:4
    x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xf, 0xf, true);   // row_shr:8
    x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xa, 0xf, false);  // row_bcast:15 into rows 1 and 3
    x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xc, 0xf, false);  // row_bcast:31 into rows 2 and 3
    return x;
}

// Descending bitonic sort of one value per lane across the wave; returns this lane's sorted value.
__device__ __forceinline__ uint32_t wave_sort_desc(uint32_t v) {
    const int l = lane_id();
#pragma unroll
    for (int size = 2; size <= 64; size <<= 1) {
#pragma unroll
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            const uint32_t w = static_cast<uint32_t>(__shfl_xor(static_cast<int>(v), stride));
            const bool desc_block = ((l & size) == 0);
            const bool lower = ((l & stride) == 0);
            // In a descending block the lower lane keeps the larger value.
            const bool keep_max = (lower == desc_block);
            v = keep_max ? max(v, w) : min(v, w);
        }
    }
    return v;
}

struct SelShared {
    uint32_t ckey[kCap];
    int32_t cidx[kCap];
    uint32_t hist[256];
    uint32_t whist[kSelWaves][256];  // per-wave bound-refinement histograms; afterwards the threshold bin's keys
    uint32_t tau_key;                // workgroup-wide lower bound of the K-th largest key (only ever raised)
    uint32_t sortbuf[kMaxTopK];
    float fred[kSelWaves];
    uint32_t ured[kSelWaves];
    uint64_t u64red[kSelWaves];
    int wcount[kSelWaves];
    int count;
    int overflow;
    int found;       // the position belongs to a batch row (fused accept)
    int last;        // this workgroup finishes its batch row (fused accept)
    uint32_t sel_digit, sel_remaining, sel_greater, sel_equal;
    float fast_m, fast_z, fast_theta;  // row statistics of the wave-0 epilogue
    uint32_t wmax[kSelWaves];          // largest key of each wave's list
    uint32_t wlo[kSelWaves];           // each wave's final lower bound of the K-th largest key
    int bin_count;                     // keys of the threshold's histogram bin
    int64_t loc[4];  // b, j, L, start
    int64_t fin_n;
    PosRecord fin_rec;
};

// Sum over the workgroup (every thread gets the result).
__device__ float block_sum(float v, SelShared& sh) {
    v = wave_sum(v);
    __syncthreads();
    if (lane_id() == 0) sh.fred[threadIdx.x >> 6] = v;
    __syncthreads();
    float t = 0.f;
    for (int w = 0; w < kSelWaves; ++w) t += sh.fred[w];
    return t;
}

__device__ uint32_t block_max_u32(uint32_t v, SelShared& sh) {
    v = wave_max_u32(v);
    __syncthreads();
    if (lane_id() == 0) sh.ured[threadIdx.x >> 6] = v;
    __syncthreads();
    uint32_t t = 0;
    for (int w = 0; w < kSelWaves; ++w) t = max(t, sh.ured[w]);
    return t;
}

__device__ uint64_t block_max_u64(uint64_t v, SelShared& sh) {
    v = wave_max_u64(v);
    __syncthreads();
    if (lane_id() == 0) sh.u64red[threadIdx.x >> 6] = v;
    __syncthreads();
    uint64_t t = 0;
    for (int w = 0; w < kSelWaves; ++w) t = sh.u64red[w] > t ? sh.u64red[w] : t;
    return t;
}

// One radix-select pass: after every key of the current prefix has been counted into sh.hist, wave 0 picks the
// digit holding the remaining-th largest key. Returns nothing; updates sh.sel_* (read after the barrier).
__device__ void radix_pick_digit(SelShared& sh) {
    if ((threadIdx.x >> 6) == 0) {
        const int l = lane_id();
        // lane l holds bins 4l .. 4l+3
        uint32_t h[4];
        uint32_t tot = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            h[i] = sh.hist[4 * l + i];
            tot += h[i];
        }
        // exclusive suffix sum over lanes (counts in bins of higher lanes) = total - inclusive prefix
        const int incl = wave_scan_incl_dpp(static_cast<int>(tot));
        uint32_t above = static_cast<uint32_t>(__builtin_amdgcn_readlane(incl, 63) - incl);  // bins of lanes > l
        const uint32_t rem = sh.sel_remaining;
#pragma unroll
        for (int i = 3; i >= 0; --i) {
            if (above < rem && rem <= above + h[i]) {
                sh.sel_digit = static_cast<uint32_t>(4 * l + i);
                sh.sel_remaining = rem - above;
                sh.sel_greater += above;
                sh.sel_equal = h[i];
            }
            above += h[i];
        }
    }
}

// rank-th largest key (1-based) among the keys produced by for_each(fn) (each thread visits its share and calls
// fn(key)). Also returns how many keys are greater / equal. Every thread gets the results.
template <class ForEach>
__device__ uint32_t radix_select(ForEach for_each, uint32_t rank, SelShared& sh, uint32_t* n_greater,
                                 uint32_t* n_equal) {
    uint32_t prefix = 0, mask = 0;
    __syncthreads();
    if (threadIdx.x == 0) {
        sh.sel_remaining = rank;
        sh.sel_greater = 0;
        sh.sel_equal = 0;
        sh.sel_digit = 0;
    }
#pragma unroll 1
    for (int pass = 0; pass < 4; ++pass) {
        const int shift = 24 - 8 * pass;
        for (int i = threadIdx.x; i < 256; i += blockDim.x) sh.hist[i] = 0;
        __syncthreads();
        for_each([&](uint32_t key) {
            if ((key & mask) == prefix) atomicAdd(&sh.hist[(key >> shift) & 255u], 1u);
        });
        __syncthreads();
        radix_pick_digit(sh);
        __syncthreads();
        prefix |= sh.sel_digit << shift;
        mask |= 255u << shift;
    }
    *n_greater = sh.sel_greater;
    *n_equal = sh.sel_equal;
    return prefix;
}

// Descending bitonic sort of sh.sortbuf[0..n) (n <= kMaxTopK), padding with 0 keys.
__device__ void block_sort_desc(SelShared& sh, int n) {
    int p = 64;
    while (p < n) p <<= 1;
    for (int i = n + threadIdx.x; i < p; i += blockDim.x) sh.sortbuf[i] = 0u;
    __syncthreads();
    for (int size = 2; size <= p; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            for (int i = threadIdx.x; i < p / 2; i += blockDim.x) {
                const int lo = 2 * i - (i & (stride - 1));
                const int hi = lo + stride;
                const uint32_t a = sh.sortbuf[lo], b = sh.sortbuf[hi];
                const bool desc = ((lo & size) == 0);
                if (desc ? (a < b) : (a > b)) {
                    sh.sortbuf[lo] = b;
                    sh.sortbuf[hi] = a;
                }
            }
            __syncthreads();
        }
    }
}


// Row locator of the fused accept: position t -> batch row b, draft index j, verified length L, first position.
__device__ void locate(const SelArgs& a, int64_t t, SelShared& sh) {
    if (a.lens == nullptr) {
        if (threadIdx.x == 0) {
            const int64_t L = a.k + 1;
            sh.loc[0] = t / L;
            sh.loc[1] = t % L;
            sh.loc[2] = L;
            sh.loc[3] = (t / L) * L;
            sh.found = (t / L) < a.batch;
        }
        __syncthreads();
        return;
    }
    int64_t carry = 0;
    for (int64_t base = 0; base < a.batch; base += blockDim.x) {
        const int64_t i = base + threadIdx.x;
        const int64_t L = i < a.batch ? a.lens[i] : 0;
        int64_t incl = wave_scan_incl_i64(L);
        // wave totals -> exclusive offsets
        __shared__ int64_t wtot[kSelWaves];
        if (lane_id() == 63) wtot[threadIdx.x >> 6] = incl;
        __syncthreads();
        int64_t off = carry;
        for (int w = 0; w < (int)(threadIdx.x >> 6); ++w) off += wtot[w];
        int64_t total = 0;
        for (int w = 0; w < kSelWaves; ++w) total += wtot[w];
        incl += off;
        const int64_t start = incl - L;
        __syncthreads();
        if (i < a.batch && L > 0 && t >= start && t < incl) {
            sh.loc[0] = i;
            sh.loc[1] = t - start;
            sh.loc[2] = L;
            sh.loc[3] = start;
            sh.found = 1;
        }
        carry += total;
    }
    __syncthreads();
}

// Elements per 16-byte piece of a logit row.
template <int DT>
constexpr int piece_elems() { return DT == NVS_DTYPE_F32 ? 4 : 8; }

// One batch of this thread's values: elements e0 + (i * kSelThreads + thread) * W + c, W elements per 16-byte
// piece. Branch-free, so the compiler can keep several batches of loads in flight (a branch around a load makes
// it wait for every outstanding load at the join). VEC (16-byte aligned rows, vocab a multiple of W): one
// streaming 16-byte load per piece from an address clamped into the row; otherwise element loads from clamped
// indices. Elements past the vocabulary read as NaN, which every filter rejects.
template <int DT, bool VEC, bool MASK = true>
__device__ __forceinline__ void load_vals(const void* row, int64_t e0, int64_t vocab, float (&v)[kVpt]) {
    constexpr int W = piece_elems<DT>();
#pragma unroll
    for (int i = 0; i < kVpt / W; ++i) {
        const int64_t e = e0 + (static_cast<int64_t>(i) * kSelThreads + threadIdx.x) * W;
        if constexpr (VEC) {
            const int64_t ec = min(e, vocab - W);
            if constexpr (DT == NVS_DTYPE_F32) {
                const f32x4 x = __builtin_nontemporal_load(
                    reinterpret_cast<const f32x4*>(static_cast<const float*>(row) + ec));
                v[4 * i] = x.x;
                v[4 * i + 1] = x.y;
                v[4 * i + 2] = x.z;
                v[4 * i + 3] = x.w;
            } else {
                const u32x4 x = __builtin_nontemporal_load(
                    reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(row) + ec));
                const uint32_t w[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    if constexpr (DT == NVS_DTYPE_BF16) {
                        v[8 * i + 2 * c] = nvs::bf16_bits_to_float(static_cast<uint16_t>(w[c] & 0xffffu));
                        v[8 * i + 2 * c + 1] = nvs::bf16_bits_to_float(static_cast<uint16_t>(w[c] >> 16));
                    } else {
                        v[8 * i + 2 * c] = nvs::f16_bits_to_float(static_cast<uint16_t>(w[c] & 0xffffu));
                        v[8 * i + 2 * c + 1] = nvs::f16_bits_to_float(static_cast<uint16_t>(w[c] >> 16));
                    }
                }
            }
            if constexpr (MASK) {
#pragma unroll
                for (int c = 0; c < W; ++c) v[W * i + c] = (e < vocab) ? v[W * i + c] : NAN;
            }
        } else {
#pragma unroll
            for (int c = 0; c < W; ++c) {
                const float x = nvs::load_as_float<DT>(row, min(e + c, vocab - 1));
                v[W * i + c] = (e + c < vocab) ? x : NAN;
            }
        }
    }
}

// Element index of value slot vi of this thread within the batch starting at e0.
template <int DT>
__device__ __forceinline__ int64_t val_index(int64_t e0, int vi) {
    if constexpr (DT == NVS_DTYPE_F32) {
        return e0 + (static_cast<int64_t>(vi >> 2) * kSelThreads + threadIdx.x) * 4 + (vi & 3);
    } else {
        return e0 + (static_cast<int64_t>(vi >> 3) * kSelThreads + threadIdx.x) * 8 + (vi & 7);
    }
}

__device__ __forceinline__ float scale_logit(float x, float temp, bool unit_temp) {
    return unit_temp ? x : x / temp;
}

// The bin of a 256-bin histogram (bins in increasing key order) that holds the rank-th largest (1-based) of the
// counted keys, and that key's rank within the bin, found by one wave (every lane gets both).
__device__ __forceinline__ void wave_pick_bin(const uint32_t* hist, uint32_t rank, uint32_t& bin, uint32_t& rem) {
    const int l = lane_id();
    uint32_t h[4];
    uint32_t tot = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        h[i] = hist[4 * l + i];
        tot += h[i];
    }
    // keys in bins of lanes > l: the total minus the inclusive prefix
    const int incl = wave_scan_incl_dpp(static_cast<int>(tot));
    uint32_t above = static_cast<uint32_t>(__builtin_amdgcn_readlane(incl, 63) - incl);
    int found_bin = -1;
    uint32_t found_rem = 0;
#pragma unroll
    for (int i = 3; i >= 0; --i) {
        if (found_bin < 0 && above < rank && rank <= above + h[i]) {
            found_bin = 4 * l + i;
            found_rem = rank - above;
        }
        above += h[i];
    }
    const uint64_t who = __ballot(found_bin >= 0);
    const int src = who ? static_cast<int>(__ffsll(static_cast<long long>(who))) - 1 : 0;
    bin = static_cast<uint32_t>(__shfl(found_bin, src));
    rem = static_cast<uint32_t>(__shfl(static_cast<int>(found_rem), src));
}

// Integer sum over the wave (every lane gets it), through the DPP reduction of wave_sum's shape.
__device__ __forceinline__ int wave_sum_i32(int v) {
    v += static_cast<int>(dpp_u32<0x128, 0xf>(0u, static_cast<uint32_t>(v)));
    v += static_cast<int>(dpp_u32<0x124, 0xf>(0u, static_cast<uint32_t>(v)));
    v += static_cast<int>(dpp_u32<0x122, 0xf>(0u, static_cast<uint32_t>(v)));
    v += static_cast<int>(dpp_u32<0x121, 0xf>(0u, static_cast<uint32_t>(v)));
    v += static_cast<int>(dpp_u32<0x142, 0xa>(0u, static_cast<uint32_t>(v)));
    v += static_cast<int>(dpp_u32<0x143, 0xc>(0u, static_cast<uint32_t>(v)));
    return __builtin_amdgcn_readlane(v, 63);
}

// Key of a value for selection; NaN padding (past the vocabulary) maps to 0, below every real value.
__device__ __forceinline__ uint32_t sel_key(float s) { return (s != s) ? 0u : nvs::float_key(s); }

// Append the values of this thread with key >= tau_key to the candidate list.
template <int DT>
__device__ __forceinline__ void append_candidates(SelShared& sh, const uint32_t (&keys)[kVpt], int64_t e0,
                                                  uint32_t tau_key) {
    uint64_t bal[kVpt];
    int tot = 0;
#pragma unroll
    for (int vi = 0; vi < kVpt; ++vi) {
        const bool pass = keys[vi] != 0u && keys[vi] >= tau_key;
        bal[vi] = __ballot(pass);
        tot += __popcll(bal[vi]);
    }
    if (tot == 0) return;
    int base = 0;
    if (lane_id() == 0) base = atomicAdd(&sh.count, tot);
    base = __shfl(base, 0);
    const uint64_t below = (lane_id() == 0) ? 0ull : (~0ull >> (64 - lane_id()));
    int run = 0;
#pragma unroll
    for (int vi = 0; vi < kVpt; ++vi) {
        if ((bal[vi] >> lane_id()) & 1ull) {
            const int pos = base + run + __popcll(bal[vi] & below);
            if (pos < kCap) {
                sh.ckey[pos] = keys[vi];
                sh.cidx[pos] = static_cast<int32_t>(val_index<DT>(e0, vi));
            } else {
                sh.overflow = 1;
            }
        }
        run += __popcll(bal[vi]);
    }
}

// Threshold of truncate_logits (spec_sampler.py:72-96) from the sorted top `rank` keys in sh.sortbuf:
// rank = min(max(top_k, 1), K); ranks >= rank are -inf among the K candidates; with top-p the nucleus softmax
// over the candidates, mass_before = cumsum - nucleus, kept = #(mass_before < top_p), p_threshold =
// candidates[kept - 1]. Returns max(candidates[rank-1], p_threshold).
__device__ float top_p_threshold(SelShared& sh, int rank, int K, float top_p, float thr) {
    __shared__ float result;
    if ((threadIdx.x >> 6) == 0) {
        const int l = lane_id();
        const float m = nvs::key_float(sh.sortbuf[0]);
        const int per = (rank + 63) / 64;
        // each lane's entries r = l * per + i, recomputed in every loop below rather than kept in a per-lane array
        // (indexed by a runtime i it would live in private memory); expf of the same input gives the same bits
        auto entry = [&](int i) {
            const int r = l * per + i;
            return (r < rank) ? expf(nvs::key_float(sh.sortbuf[r]) - m) : 0.f;
        };
        float lsum = 0.f;
        for (int i = 0; i < per && i < 16; ++i) lsum += entry(i);
        const float total = wave_sum(lsum);
        // The nucleus cumsum as torch's CPU cumsum of fp32 computes it: accumulated in double, each prefix rounded
        // to float, then the float subtraction of the entry (spec_sampler.py:91). An fp32 running sum reaches 1.0
        // early on a peaked row and would cut entries the reference keeps. Local sums first, then the lanes'
        // exclusive prefix.
        double loc = 0.0;
        for (int i = 0; i < per && i < 16; ++i) loc += static_cast<double>(entry(i) / total);
        const double incl = wave_scan_incl_f64(loc);
        double run = incl - loc;
        int kept = 0;
        for (int i = 0; i < per && i < 16; ++i) {
            const int r = l * per + i;
            if (r < rank) {
                const float e = entry(i) / total;
                run += static_cast<double>(e);
                const float before = static_cast<float>(run) - e;
                kept += (before < top_p) ? 1 : 0;
            }
        }
        const float last_cum = static_cast<float>(__shfl(incl, 63));  // cumsum at rank - 1 (later entries add 0)
        int kept_all = static_cast<int>(wave_sum(static_cast<float>(kept)));
        if (last_cum < top_p) kept_all += K - rank;
        if (l == 0) {
            float p_thr = -INFINITY;
            if (kept_all >= 1 && kept_all - 1 < rank) p_thr = nvs::key_float(sh.sortbuf[kept_all - 1]);
            result = fmaxf(thr, p_thr);
        }
    }
    __syncthreads();
    return result;
}

// The same threshold computed by one wave when rank <= 64: lane l holds the l-th largest candidate key (the
// rank-th largest repeated where candidates tie with it, as top-k ranks beyond it are -inf), 0 past rank. Every
// lane gets the result.
__device__ float wave_top_p_threshold64(uint32_t key_l, int rank, int K, float top_p, float thr) {
    const int l = lane_id();
    const float m = nvs::key_float(static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(key_l))));
    const float e = (l < rank) ? expf(nvs::key_float(key_l) - m) : 0.f;
    const float total = wave_sum(e);
    const float nucleus = e / total;
    // the cumsum accumulated in double and rounded per prefix, as torch's CPU cumsum of fp32 (see top_p_threshold)
    const float cum = static_cast<float>(wave_scan_incl_f64(static_cast<double>(nucleus)));
    const float before = cum - nucleus;
    int kept_all = __popcll(__ballot(l < rank && before < top_p));
    const float last_cum = __shfl(cum, 63);   // cumsum at rank - 1 (all later entries add zero)
    if (last_cum < top_p) kept_all += K - rank;
    const uint32_t at = static_cast<uint32_t>(__shfl(static_cast<int>(key_l), max(kept_all - 1, 0)));
    const float p_thr = (kept_all >= 1 && kept_all - 1 < rank) ? nvs::key_float(at) : -INFINITY;
    return fmaxf(thr, p_thr);
}

struct RowStats {
    float m, z, theta;
    bool dense;   // kept set not held in the candidate list
};

// Sum over the workgroup in double, in a fixed order (every thread gets the result).
__device__ double block_sum_f64(double v, SelShared& sh) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    __syncthreads();
    if (lane_id() == 0) sh.u64red[threadIdx.x >> 6] = static_cast<uint64_t>(__double_as_longlong(v));
    __syncthreads();
    double t = 0.0;
    for (int w = 0; w < kSelWaves; ++w) t += __longlong_as_double(static_cast<long long>(sh.u64red[w]));
    return t;
}

// ---------------------------------------------------------------- windows wider than the candidate lists
// A row whose top-k window holds more than kMaxTopK values (top_k up to the vocabulary, sampling_params.py:15-16)
// keeps nothing in LDS: the rank-th largest value comes from a radix select over the row, the top-p threshold from
// a radix descent over nucleus mass (below), and the softmax sum and every later use re-read the row.

// Nucleus probabilities (in [0, 1]) are summed in 64-bit fixed point with 62 fraction bits: integer sums are exact
// whatever order the atomics land in, so the descent is deterministic; a probability below 2^-62 adds nothing.
constexpr double kMassScale = 4611686018427387904.0;   // 2^62

__device__ __forceinline__ unsigned long long mass_fixed(float n) {
    return static_cast<unsigned long long>(static_cast<double>(n) * kMassScale);
}

// Whether top-p keeps the first rank holding a value of nucleus probability n, when the ranks before it hold
// nucleus mass `before` (fixed point): mass_before = cumsum - nucleus (spec_sampler.py:90-91), the cumsum as torch's
// CPU cumsum of fp32 forms it (a double running sum rounded to float at each prefix), tested < top_p.
__device__ __forceinline__ bool nucleus_keeps(unsigned long long before, float n, float top_p) {
    const double cum = static_cast<double>(before) / kMassScale + static_cast<double>(n);
    return static_cast<float>(cum) - n < top_p;
}

// Top-p threshold of a wide window without sorting it. The nucleus is the softmax over the window's `rank` values:
// the n_gt values above thr plus rank - n_gt copies of thr (the window's ranks past top_k are -inf,
// spec_sampler.py:82-89), and kept = #(ranks whose mass_before < top_p); the threshold is the kept-th largest.
// mass_before grows with the rank, so that is the smallest window value whose first rank is kept. A radix descent
// over the window's keys finds it: per 8-bit digit, each bin's nucleus mass, key count and largest key; the bin
// whose largest key is kept and that lies lowest holds it, and the mass of the bins above carries into the next
// digit. Returns thr when no rank is kept (top_p <= 0).
template <class ForEach>
__device__ float wide_top_p_threshold(ForEach for_each, uint32_t thr_key, uint32_t n_gt, int rank, float m,
                                      float top_p, SelShared& sh) {
    const float thr = nvs::key_float(thr_key);
    const uint32_t copies = static_cast<uint32_t>(rank) - n_gt;
    // the nucleus denominator over up to the whole vocabulary, summed in double: an fp32 sum of 10^5 terms would
    // carry relative errors near 1e-6, the size of the mass differences the top-p test resolves
    double tot_d = 0.0;
    for_each([&](uint32_t key) {
        if (key > thr_key) tot_d += static_cast<double>(expf(nvs::key_float(key) - m));
    });
    tot_d = block_sum_f64(tot_d, sh) + static_cast<double>(copies) * static_cast<double>(expf(thr - m));
    const float tot = static_cast<float>(tot_d);
    // the refinement histograms' space is free on this path: masses, then largest keys; counts in sh.hist
    unsigned long long* hmass = reinterpret_cast<unsigned long long*>(&sh.whist[0][0]);
    uint32_t* hmax = &sh.whist[4][0];
    uint32_t* hcnt = sh.hist;
    __shared__ unsigned long long desc_above;
    __shared__ uint32_t desc_digit;
    __shared__ int desc_found;
    uint32_t prefix = 0u, mask = 0u;
    unsigned long long above = 0ull;   // nucleus mass of the window's keys above the current digit's range
#pragma unroll 1
    for (int pass = 0; pass < 4; ++pass) {
        const int shift = 24 - 8 * pass;
        for (int i = threadIdx.x; i < 256; i += blockDim.x) {
            hmass[i] = 0ull;
            hmax[i] = 0u;
            hcnt[i] = 0u;
        }
        __syncthreads();
        for_each([&](uint32_t key) {
            if (key <= thr_key || (key & mask) != prefix) return;   // thr's copies are counted below
            const uint32_t bin = (key >> shift) & 255u;
            atomicAdd(&hmass[bin], mass_fixed(expf(nvs::key_float(key) - m) / tot));
            atomicAdd(&hcnt[bin], 1u);
            atomicMax(&hmax[bin], key);
        });
        if (threadIdx.x == 0 && (thr_key & mask) == prefix && copies > 0u) {
            const uint32_t bin = (thr_key >> shift) & 255u;
            atomicAdd(&hmass[bin], static_cast<unsigned long long>(copies) * mass_fixed(expf(thr - m) / tot));
            atomicAdd(&hcnt[bin], copies);
            atomicMax(&hmax[bin], thr_key);
        }
        __syncthreads();
        if (threadIdx.x < 64) {
            // lane l holds bins 4l .. 4l+3; the bins of higher lanes lie above them
            const int l = lane_id();
            unsigned long long mb[4];
            uint32_t cb[4], kb[4];
            unsigned long long lane_mass = 0ull;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                mb[i] = hmass[4 * l + i];
                cb[i] = hcnt[4 * l + i];
                kb[i] = hmax[4 * l + i];
                lane_mass += mb[i];
            }
            const int64_t incl = wave_scan_incl_i64(static_cast<int64_t>(lane_mass));
            const int64_t total = __shfl(incl, 63);
            unsigned long long run = above + static_cast<unsigned long long>(total - incl);
            uint32_t lowest = 256u;
            unsigned long long lowest_above = 0ull;
#pragma unroll
            for (int i = 3; i >= 0; --i) {
                if (cb[i] > 0u && nucleus_keeps(run, expf(nvs::key_float(kb[i]) - m) / tot, top_p)) {
                    lowest = static_cast<uint32_t>(4 * l + i);
                    lowest_above = run;
                }
                run += mb[i];
            }
            const uint32_t best = 256u - wave_max_u32(256u - lowest);
            if (best < 256u && lowest == best) {
                desc_above = lowest_above;
                desc_digit = best;
            }
            if (l == 0) desc_found = best < 256u ? 1 : 0;
        }
        __syncthreads();
        if (!desc_found) return thr;
        above = desc_above;
        prefix |= desc_digit << shift;
        mask |= 255u << shift;
        __syncthreads();   // every thread has read the digit before the next pass rewrites it
    }
    return nvs::key_float(prefix);
}

// Row statistics of a wide window: the rank-th largest value by a radix select over the row, the row maximum, the
// top-p threshold as above, and the softmax sum over the kept values; the kept set stays in the row (dense).
template <int DT, bool VEC>
__device__ RowStats wide_row_stats(const SelArgs& a, const void* row, float temp, bool unit_temp, int rank,
                                   float top_p, SelShared& sh) {
    auto for_each = [&](auto&& fn) {
        for (int64_t e0 = 0; e0 < a.vocab; e0 += kBatch) {
            float v[kVpt];
            load_vals<DT, VEC>(row, e0, a.vocab, v);
#pragma unroll
            for (int vi = 0; vi < kVpt; ++vi) {
                const uint32_t key = sel_key(scale_logit(v[vi], temp, unit_temp));
                if (key != 0u) fn(key);
            }
        }
    };
    uint32_t n_gt = 0, n_eq = 0;
    const uint32_t thr_key = radix_select(for_each, static_cast<uint32_t>(rank), sh, &n_gt, &n_eq);
    uint32_t mk = 0u;
    for_each([&](uint32_t key) { mk = max(mk, key); });
    mk = block_max_u32(mk, sh);
    RowStats rs;
    rs.m = nvs::key_float(mk);
    rs.theta = nvs::key_float(thr_key);
    if (a.has_top_p) rs.theta = wide_top_p_threshold(for_each, thr_key, n_gt, rank, rs.m, top_p, sh);
    const uint32_t theta_key = nvs::float_key(rs.theta);
    double z = 0.0;   // in double, as the nucleus denominator above
    for_each([&](uint32_t key) {
        if (key >= theta_key) z += static_cast<double>(expf(nvs::key_float(key) - rs.m));
    });
    rs.z = static_cast<float>(block_sum_f64(z, sh));
    rs.dense = true;
    return rs;
}

// Full-row exact path (candidate list overflowed): radix select on the row, then rebuild the candidate list.
// WIDE: the kernel serves windows wider than the lists (wide_row_stats), compiled only into the select kernels
// launched for such batches so that the others keep their registers.
template <int DT, bool VEC, bool WIDE>
__device__ RowStats exact_row_stats(const SelArgs& a, const void* row, float temp, bool unit_temp,
                                    int rank, int K, float top_p, SelShared& sh) {
    if constexpr (WIDE) {
        if (rank > kMaxTopK) return wide_row_stats<DT, VEC>(a, row, temp, unit_temp, rank, top_p, sh);
    }
    auto for_each = [&](auto&& fn) {
        for (int64_t e0 = 0; e0 < a.vocab; e0 += kBatch) {
            float v[kVpt];
            load_vals<DT, VEC>(row, e0, a.vocab, v);
#pragma unroll
            for (int vi = 0; vi < kVpt; ++vi) {
                const uint32_t key = sel_key(scale_logit(v[vi], temp, unit_temp));
                if (key != 0u) fn(key);
            }
        }
    };
    uint32_t n_gt = 0, n_eq = 0;
    const uint32_t thr_key = radix_select(for_each, static_cast<uint32_t>(rank), sh, &n_gt, &n_eq);
    const bool fits = (n_gt + n_eq) <= static_cast<uint32_t>(kCap);
    // Rebuild the candidate list: everything >= thr when it fits, else only the (fewer than rank) keys above it.
    __syncthreads();
    if (threadIdx.x == 0) {
        sh.count = 0;
        sh.overflow = 0;
    }
    __syncthreads();
    const uint32_t floor_key = fits ? thr_key : thr_key + 1u;
    for (int64_t e0 = 0; e0 < a.vocab; e0 += kBatch) {
        float v[kVpt];
        load_vals<DT, VEC>(row, e0, a.vocab, v);
        uint32_t keys[kVpt];
#pragma unroll
        for (int vi = 0; vi < kVpt; ++vi) keys[vi] = sel_key(scale_logit(v[vi], temp, unit_temp));
        append_candidates<DT>(sh, keys, e0, floor_key);
    }
    __syncthreads();
    RowStats rs;
    const int n = min(sh.count, kCap);
    // max
    uint32_t mk = 0;
    for (int c = threadIdx.x; c < n; c += blockDim.x) mk = max(mk, sh.ckey[c]);
    mk = block_max_u32(mk, sh);
    if (n == 0) mk = thr_key;
    rs.m = nvs::key_float(mk);
    const float thr = nvs::key_float(thr_key);
    rs.theta = thr;
    if (a.has_top_p) {
        // sorted top rank keys: the ones above thr, then copies of thr
        // gather keys > thr into sortbuf
        __shared__ int gcount;
        if (threadIdx.x == 0) gcount = 0;
        __syncthreads();
        for (int c = threadIdx.x; c < n; c += blockDim.x) {
            if (sh.ckey[c] > thr_key) sh.sortbuf[atomicAdd(&gcount, 1)] = sh.ckey[c];
        }
        __syncthreads();
        const int g = gcount;
        block_sort_desc(sh, g);
        for (int i = g + threadIdx.x; i < rank; i += blockDim.x) sh.sortbuf[i] = thr_key;
        __syncthreads();
        rs.theta = top_p_threshold(sh, rank, K, top_p, thr);
    }
    const uint32_t theta_key = nvs::float_key(rs.theta);
    rs.dense = !(fits || rs.theta > thr);
    float z = 0.f;
    if (!rs.dense) {
        for (int c = threadIdx.x; c < n; c += blockDim.x)
            if (sh.ckey[c] >= theta_key) z += expf(nvs::key_float(sh.ckey[c]) - rs.m);
    } else {
        for (int64_t e0 = 0; e0 < a.vocab; e0 += kBatch) {
            float v[kVpt];
            load_vals<DT, VEC>(row, e0, a.vocab, v);
#pragma unroll
            for (int vi = 0; vi < kVpt; ++vi) {
                const float s = scale_logit(v[vi], temp, unit_temp);
                if (sel_key(s) >= theta_key && sel_key(s) != 0u) z += expf(s - rs.m);
            }
        }
    }
    rs.z = block_sum(z, sh);
    return rs;
}

// ---------------------------------------------------------------- q as candidate rows
// A draft row's q given as candidate rows (DSpark's candidate rows, written by nvs_markov_draw): token ids
// ids[slot * q_stride + c] with probabilities probs[...], c < q_cand, id -1 for no token. q(token) is the
// probability of the entry holding the token, 0 when none does (the reference scatters the rows over a zeroed
// [B, k, V] q, speculative.py:169-180).

// q(token) by one whole wave: every lane checks every 64th entry; the first entry holding the token wins.
__device__ float sparse_q_wave(const SelArgs& a, int64_t slot, int64_t token) {
    const int32_t* ids = a.q_ids + slot * a.q_stride;
    const float* probs = a.q_probs + slot * a.q_stride;
    const int l = lane_id();
    float found = 0.f;
    int at = 0x7fffffff;
    for (int c0 = 0; c0 < a.q_cand; c0 += 64) {
        const int c = c0 + l;
        const bool in = c < a.q_cand;
        const int32_t id = in ? ids[c] : -1;
        const float p = in ? probs[c] : 0.f;
        if (id >= 0 && id == token && c < at) {
            found = p;
            at = c;
        }
    }
    const int first = 0x7fffffff - static_cast<int>(wave_max_u32(static_cast<uint32_t>(0x7fffffff - at)));
    if (first == 0x7fffffff) return 0.f;
    const uint64_t who = __ballot(at == first);
    return __shfl(found, static_cast<int>(__ffsll(static_cast<long long>(who))) - 1);
}

// q at each lane's kSelWaves tokens: every entry of the row is broadcast across the wave (64 at a time).
__device__ void sparse_q_wave8(const SelArgs& a, int64_t slot, const int32_t (&tok)[kSelWaves],
                               float (&q)[kSelWaves]) {
    const int32_t* ids = a.q_ids + slot * a.q_stride;
    const float* probs = a.q_probs + slot * a.q_stride;
    const int l = lane_id();
    bool done[kSelWaves];
#pragma unroll
    for (int w = 0; w < kSelWaves; ++w) {
        q[w] = 0.f;
        done[w] = false;
    }
    for (int c0 = 0; c0 < a.q_cand; c0 += 64) {
        const int c = c0 + l;
        const bool in = c < a.q_cand;
        const int32_t id = in ? ids[c] : -1;
        const float p = in ? probs[c] : 0.f;
        const int n = min(64, a.q_cand - c0);
        for (int src = 0; src < n; ++src) {
            const int32_t bid = __builtin_amdgcn_readlane(id, src);
            const float bp = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(p), src));
#pragma unroll
            for (int w = 0; w < kSelWaves; ++w) {
                const bool hit = !done[w] && bid >= 0 && tok[w] == bid;
                q[w] = hit ? bp : q[w];
                done[w] = done[w] || hit;
            }
        }
    }
}

// q(token) by one thread, scanning the row (rows with more candidates than the hash holds).
__device__ float sparse_q_scan(const SelArgs& a, int64_t slot, int64_t token) {
    const int32_t* ids = a.q_ids + slot * a.q_stride;
    const float* probs = a.q_probs + slot * a.q_stride;
    for (int c = 0; c < a.q_cand; ++c)
        if (ids[c] >= 0 && ids[c] == token) return probs[c];
    return 0.f;
}

// Open-addressing hash of a row's tokens in the refinement histograms' space (free once the row statistics are
// known): keys (token + 1, 0 = empty) in the first kQHash words, probabilities in the next kQHash. At most
// kQHash / 2 entries, so every probe sequence meets an empty slot.
constexpr int kQHash = 1024;
static_assert(2 * kQHash <= kSelWaves * 256, "the hash must fit the refinement histograms");

__device__ __forceinline__ uint32_t q_hash(int64_t token) {
    return (static_cast<uint32_t>(token) * 2654435761u) >> 22;   // 10 bits
}

__device__ void build_q_hash(const SelArgs& a, int64_t slot, SelShared& sh) {
    uint32_t* keys = &sh.whist[0][0];
    uint32_t* vals = keys + kQHash;
    for (int i = threadIdx.x; i < kQHash; i += blockDim.x) keys[i] = 0u;
    __syncthreads();
    const int32_t* ids = a.q_ids + slot * a.q_stride;
    const float* probs = a.q_probs + slot * a.q_stride;
    for (int c = threadIdx.x; c < a.q_cand; c += blockDim.x) {
        const int32_t id = ids[c];
        if (id < 0) continue;
        const uint32_t key = static_cast<uint32_t>(id) + 1u;
        uint32_t h = q_hash(id);
        for (int probe = 0; probe < kQHash; ++probe) {
            const uint32_t was = atomicCAS(&keys[h], 0u, key);
            if (was == 0u) {
                vals[h] = __float_as_uint(probs[c]);
                break;
            }
            h = (h + 1u) & (kQHash - 1);
        }
    }
    __syncthreads();
}

// The row's first 128 candidates (lane and lane + 64), requested by the wave-0 finish before its threshold so that
// their round trip overlaps it; id -1 past the row's candidates.
__device__ __forceinline__ void load_q_row_head(const SelArgs& a, int64_t slot, int32_t (&id)[2], float (&pr)[2]) {
    const int32_t* ids = a.q_ids + slot * a.q_stride;
    const float* probs = a.q_probs + slot * a.q_stride;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int c = lane_id() + 64 * h;
        id[h] = c < a.q_cand ? ids[c] : -1;
        pr[h] = c < a.q_cand ? probs[c] : 0.f;
    }
}

// The same hash built by one wave alone (the wave-0 finish, while the other waves wait), from the row's first 128
// candidates already in registers and the rest loaded here: LDS operations of one wave take effect in program order,
// so the lookups that follow see every insert. Each id is in the row once, so the order of inserts does not matter.
__device__ __forceinline__ void build_q_hash_wave(const SelArgs& a, int64_t slot, SelShared& sh, int32_t id0,
                                                  float pr0, int32_t id1, float pr1) {
    uint32_t* keys = &sh.whist[0][0];
    uint32_t* vals = keys + kQHash;
    const int32_t* ids = a.q_ids + slot * a.q_stride;
    const float* probs = a.q_probs + slot * a.q_stride;
    for (int i = lane_id(); i < kQHash; i += 64) keys[i] = 0u;
    compiler_fence_s();
    auto insert = [&](int32_t id, float pr) {
        if (id < 0) return;
        const uint32_t key = static_cast<uint32_t>(id) + 1u;
        uint32_t h = q_hash(id);
        for (int probe = 0; probe < kQHash; ++probe) {
            const uint32_t was = atomicCAS(&keys[h], 0u, key);
            if (was == 0u) {
                vals[h] = __float_as_uint(pr);
                break;
            }
            h = (h + 1u) & (kQHash - 1);
        }
    };
    insert(id0, pr0);
    insert(id1, pr1);
    for (int c = lane_id() + 128; c < a.q_cand; c += 64) insert(ids[c], probs[c]);
    compiler_fence_s();
}

__device__ float q_hash_lookup(SelShared& sh, int64_t token) {
    const uint32_t* keys = &sh.whist[0][0];
    const uint32_t* vals = keys + kQHash;
    const uint32_t key = static_cast<uint32_t>(token) + 1u;
    uint32_t h = q_hash(token);
    for (int probe = 0; probe < kQHash; ++probe) {
        const uint32_t k = keys[h];
        if (k == key) return __uint_as_float(vals[h]);
        if (k == 0u) return 0.f;
        h = (h + 1u) & (kQHash - 1);
    }
    return 0.f;
}

// Finish batch row b of the fused accept (run by the workgroup whose position arrived last): the accepted prefix
// n from the positions' decisions, then the tail = the race of position start + n, which that position already ran
// over its kept set, or, for a row that does not truncate, a race over the whole vocabulary run here. The caller
// has acquired the other positions' records (count_position).
template <int DT>
__device__ __forceinline__ void finish_row(const SelArgs& a, int64_t b, int64_t start, int64_t L, SelShared& sh) {
    const int kd = a.k;
    if (threadIdx.x < 64) {
        // wave 0: lane i loads the record of position start + c0 + i, all in one round trip; the first position
        // that is rejected or cannot be accepted ends the prefix and its record gives the tail
        const int lane = threadIdx.x;
        const int64_t lim = min(min(L - 1, static_cast<int64_t>(kd)), a.n_pos - start);   // n stays <= lim
        for (int64_t c0 = 0;; c0 += 64) {
            const int64_t pos = min(start + c0 + lane, a.n_pos - 1);
            const PosRecord r = load_record(a.rec + pos);
            const bool stop = (c0 + lane >= lim) || !r.acc;
            const uint64_t bal = __ballot(stop);
            if (bal == 0ull) continue;   // all 64 accepted: the next 64
            const int first = __ffsll(static_cast<long long>(bal)) - 1;
            if (lane == first) {
                const int64_t n = c0 + first;
                sh.fin_n = n;
                sh.fin_rec = r;
                if (!(r.flags & kFlagDense)) {   // the tail is that position's own race: the row is done
                    a.n_accept[b] = n;
                    a.tail[b] = r.race;
                    a.counters[b] = 0;   // ready for the next call
                    if (a.dense_race != nullptr) a.dense_race[b].valid = 0;
                } else if (a.dense_race != nullptr) {
                    // the race over the whole vocabulary runs in the dense race kernels, spread over the chip
                    DenseRace d;
                    d.pos = min(start + n, a.n_pos - 1);
                    d.qrow = (n == L - 1) ? -1 : b * kd + (n < kd - 1 ? n : kd - 1);
                    d.m = r.m;
                    d.z = r.z;
                    d.temp = r.temp;
                    d.valid = 1;
                    a.dense_race[b] = d;
                    a.n_accept[b] = n;
                    a.counters[b] = 0;
                }
            }
            break;
        }
    }
    __syncthreads();
    const int64_t n = sh.fin_n;
    const PosRecord r = sh.fin_rec;
    if ((r.flags & kFlagDense) && a.dense_race == nullptr) {
        const int64_t pos = min(start + n, a.n_pos - 1);
        const bool bonus = (n == L - 1);
        const int64_t qn = n < kd - 1 ? n : kd - 1;
        const int64_t qslot = b * kd + qn;
        // q of the rejected draft: the dense row, or its candidate rows (hashed in LDS when they fit)
        const bool sparse = a.q_ids != nullptr;
        const bool hashed = sparse && !bonus && a.q_cand <= kQHash / 2;
        if (hashed) build_q_hash(a, qslot, sh);
        auto q_at = [&](int64_t i) -> float {
            if (!sparse) return a.q[qslot * a.vocab + i];
            return hashed ? q_hash_lookup(sh, i) : sparse_q_scan(a, qslot, i);
        };
        const float* erow = a.noise + b * a.vocab;
        const char* row = static_cast<const char*>(a.logits) + pos * a.row_stride * nvs::dtype_size(DT);
        const uint32_t theta_key = r.theta == -INFINITY ? 0u : nvs::float_key(r.theta);
        const float mu = (r.m == -INFINITY) ? 0.f : r.m;
        const bool unit_temp = (r.temp == 1.f);
        uint64_t best = 0;
        for (int64_t i = threadIdx.x; i < a.vocab; i += blockDim.x) {
            const float sc = scale_logit(nvs::load_as_float<DT>(row, i), r.temp, unit_temp);
            const float p = (sel_key(sc) >= theta_key && sc == sc) ? expf(sc - mu) / r.z : 0.f;
            const float w = bonus ? p : fmaxf(p - q_at(i), 0.f);
            const float score = w / erow[i];
            const uint64_t k64 = (static_cast<uint64_t>(nvs::float_key(score)) << 32) |
                                 static_cast<uint64_t>(0xffffffffu - static_cast<uint32_t>(i));
            best = best > k64 ? best : k64;
        }
        best = block_max_u64(best, sh);
        if (threadIdx.x == 0) {
            a.n_accept[b] = n;
            a.tail[b] = static_cast<int64_t>(0xffffffffu - static_cast<uint32_t>(best));
            a.counters[b] = 0;  // ready for the next call
        }
    }
}

// Positions of a batch row that has L verified positions from `start` and was located by a workgroup (L >= 1,
// start < n_pos): each of them counts itself once, so the row's counter reaches exactly this and is reset by the
// finish. Lengths that run past the logits (lens summing to more than n_pos) count only the positions that exist,
// so the counter never stays non-zero for the next call.
__device__ __forceinline__ int64_t row_positions(const SelArgs& a, int64_t start, int64_t L) {
    return min(L, a.n_pos - start);
}

// Count a finished position of batch row b on the row's counter; the position that counts last finishes the row.
// Returns whether this position counted last. The caller stored its record with store_record: the wait below
// holds the add back until those stores are performed at the coherence point, and the finishing workgroup issues
// its record loads (load_record, also at the coherence point) only after its own add has returned, so it reads
// every record of the row.
__device__ __forceinline__ bool count_position(int* counter, int64_t n_positions) {
    __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0): every store of this wave has completed
    const int before = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return before == static_cast<int>(n_positions) - 1;
}

// The end of one vocabulary chunk of a race spread over (row, chunk) workgroups, run by wave 0 of the chunk's
// workgroup: lane 0 publishes the chunk's best key to the row's partials at the coherence point and counts the
// chunk on the row's counter (count_position); the workgroup that counts last reads every chunk's key of the row
// (one load per lane, at the coherence point), resets the counter for the next call and returns true with the
// row's best key in winner. Every lane of wave 0 must call it; the result is uniform over the wave.
__device__ __forceinline__ bool finish_race_chunk(uint64_t* row_partials, int n_chunks, int c, uint64_t key,
                                                  int* counter, uint64_t& winner) {
    const int lane = threadIdx.x & 63;
    int last = 0;
    if (lane == 0) {
        __hip_atomic_store(row_partials + c, key, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        last = count_position(counter, n_chunks) ? 1 : 0;
    }
    last = __builtin_amdgcn_readfirstlane(last);
    if (!last) return false;
    uint64_t best = 0;
    for (int j = lane; j < n_chunks; j += 64) {
        const uint64_t v = __hip_atomic_load(row_partials + j, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        best = best > v ? best : v;
    }
    winner = wave_max_u64(best);
    if (lane == 0) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return true;
}

// ---------------------------------------------------------------- Markov draw (DSpark candidate rows)

// (key, index) pairs of a Markov draw: key << 32 | ~index, so that a descending sort orders by value, then by
// index ascending. They reuse the space of ckey and cidx (contiguous, 64 KB).
constexpr int kPairCap = kCap;
// Candidates of a Markov row: the pairs must hold the values above the threshold (fewer than max_top_k <= 1024)
// and the ties taken after them.
constexpr int kMaxCandidates = kPairCap - kMaxTopK;

__device__ __forceinline__ uint64_t* pair_buf(SelShared& sh) { return reinterpret_cast<uint64_t*>(sh.ckey); }

// Descending bitonic sort of buf[0..n) (n <= kPairCap), padded with zeros to a power of two.
__device__ void block_sort_desc_u64(uint64_t* buf, int n) {
    int p = 64;
    while (p < n) p <<= 1;
    for (int i = n + threadIdx.x; i < p; i += blockDim.x) buf[i] = 0ull;
    __syncthreads();
    for (int size = 2; size <= p; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            for (int i = threadIdx.x; i < p / 2; i += blockDim.x) {
                const int lo = 2 * i - (i & (stride - 1));
                const int hi = lo + stride;
                const uint64_t x = buf[lo], y = buf[hi];
                const bool desc = ((lo & size) == 0);
                if (desc ? (x < y) : (x > y)) {
                    buf[lo] = y;
                    buf[hi] = x;
                }
            }
            __syncthreads();
        }
    }
}

// Exclusive prefix over the workgroup in thread order; *total gets the sum (every thread).
__device__ int block_scan_excl(int v, SelShared& sh, int* total) {
    const int incl = wave_scan_incl_dpp(v);
    __syncthreads();
    if (lane_id() == 63) sh.wcount[threadIdx.x >> 6] = incl;
    __syncthreads();
    int before = 0, all = 0;
    for (int w = 0; w < kSelWaves; ++w) {
        const int c = sh.wcount[w];
        before += (w < static_cast<int>(threadIdx.x >> 6)) ? c : 0;
        all += c;
    }
    *total = all;
    return before + incl - v;
}

// One past the index of the need-th value (1-based, in index order) whose key equals tie_key; the vocabulary size
// when the row has fewer. Within a batch, value slot vi of thread x holds element
// e0 + ((vi / W) * kSelThreads + x) * W + vi % W, so index order is (slot group, thread, slot in group).
template <int DT, bool VEC>
__device__ int64_t nth_tie_end(const SelArgs& a, const char* row, float temp, bool unit_temp, uint32_t tie_key,
                               int need, SelShared& sh) {
    constexpr int W = piece_elems<DT>();
    if (need <= 0) return 0;
    int seen = 0;
    for (int64_t e0 = 0; e0 < a.vocab; e0 += kBatch) {
        float v[kVpt];
        load_vals<DT, VEC>(row, e0, a.vocab, v);
#pragma unroll
        for (int g = 0; g < kVpt / W; ++g) {
            int mine = 0;
#pragma unroll
            for (int c = 0; c < W; ++c) mine += (sel_key(scale_logit(v[g * W + c], temp, unit_temp)) == tie_key);
            int total = 0;
            const int before = block_scan_excl(mine, sh, &total);
            if (seen + total >= need) {
                // the need-th tie is in this slot group: the thread holding it reports its index
                int r = seen + before;
#pragma unroll
                for (int c = 0; c < W; ++c) {
                    if (sel_key(scale_logit(v[g * W + c], temp, unit_temp)) == tie_key && ++r == need)
                        sh.loc[3] = val_index<DT>(e0, g * W + c) + 1;
                }
                __syncthreads();
                return sh.loc[3];
            }
            seen += total;
        }
    }
    return a.vocab;
}

// The end of a Markov draw, once the candidates pairs[0..nc) (value descending) are kept: probabilities
// exp(s - m) / Z with Z over the candidates, the race argmax_c p_c / noise[c] (first rank on ties, rank 0 when every
// score is zero), the candidate row (id -1 and probability 0 past the candidates) and the drawn token.
__device__ void markov_emit(const uint64_t* pairs, int nc, int C, const float* noise, int32_t* ids, float* probs,
                            int64_t* draw, SelShared& sh) {
    const float m = nc > 0 ? nvs::key_float(static_cast<uint32_t>(pairs[0] >> 32)) : 0.f;
    float z = 0.f;
    for (int c = threadIdx.x; c < nc; c += blockDim.x)
        z += expf(nvs::key_float(static_cast<uint32_t>(pairs[c] >> 32)) - m);
    z = block_sum(z, sh);
    uint64_t best = 0;
    for (int c = threadIdx.x; c < C; c += blockDim.x) {
        float p = 0.f;
        int32_t id = -1;
        if (c < nc) {
            const uint64_t pr = pairs[c];
            p = expf(nvs::key_float(static_cast<uint32_t>(pr >> 32)) - m) / z;
            id = static_cast<int32_t>(0xffffffffu - static_cast<uint32_t>(pr));
        }
        ids[c] = id;
        probs[c] = p;
        const float score = p / noise[c];
        const uint64_t k64 = (static_cast<uint64_t>(nvs::float_key(score)) << 32) |
                             static_cast<uint64_t>(0xffffffffu - static_cast<uint32_t>(c));
        best = best > k64 ? best : k64;
    }
    best = block_max_u64(best, sh);
    if (threadIdx.x == 0) {
        const float score = nvs::key_float(static_cast<uint32_t>(best >> 32));
        const int win = (score > 0.f) ? static_cast<int>(0xffffffffu - static_cast<uint32_t>(best)) : 0;
        *draw = win < nc ? static_cast<int64_t>(0xffffffffu - static_cast<uint32_t>(pairs[win])) : int64_t{0};
    }
}

// DSpark's Markov row (speculative.py:173-180) for one position, after the row statistics: the candidates are
// the kept values (key >= theta_key) in (value descending, index ascending) order, at most n_cand of them; their
// probabilities exp(s - m) / Z with Z over the candidates; the race argmax_c p_c / noise[c] by candidate rank, the
// first rank on ties, rank 0 when every score is zero; the drawn token and the sparse row (ids, probs), with
// id -1 and probability 0 past the candidates.
// Where the kept values are when the tail starts: the wave-0 finish's short list (sortbuf: keys, then indices at
// 512), the lanes' lists (ckey / cidx, sh.count entries), or only in the row (after the exact path).
enum KeptSource { kKeptInRow = 0, kKeptInShortList = 1, kKeptInLists = 2 };

template <int DT, bool VEC>
__device__ void markov_tail(const SelArgs& a, int64_t t, const char* row, float temp, bool unit_temp,
                            uint32_t theta_key, int source, SelShared& sh) {
    uint64_t* pairs = pair_buf(sh);
    const int C = a.n_cand;
    // The lists hold every value at or above the row's threshold, so the kept ones come from there without a
    // second pass over the row. Each thread takes its entries into registers before the pairs overwrite them.
    auto collect_from_lists = [&]() {
        constexpr int kPer = kCap / kSelThreads;
        uint32_t kk[kPer];
        uint32_t ii[kPer];
        const int n = source == kKeptInShortList ? sh.count : min(sh.count, kCap);
#pragma unroll
        for (int s = 0; s < kPer; ++s) {
            const int c = static_cast<int>(threadIdx.x) + s * kSelThreads;
            const bool in = c < n && (source == kKeptInLists || s == 0);
            kk[s] = in ? (source == kKeptInShortList ? sh.sortbuf[c] : sh.ckey[c]) : 0u;
            ii[s] = in ? (source == kKeptInShortList ? sh.sortbuf[kSelWaves * 64 + c]
                                                     : static_cast<uint32_t>(sh.cidx[c]))
                       : 0u;
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            sh.count = 0;
            sh.bin_count = 0;
        }
        __syncthreads();
#pragma unroll
        for (int s = 0; s < kPer; ++s) {
            const uint32_t key = kk[s];
            if (key == 0u || key < theta_key) continue;
            const int p = atomicAdd(&sh.count, 1);
            if (key > theta_key) atomicAdd(&sh.bin_count, 1);
            pairs[p] = (static_cast<uint64_t>(key) << 32) | (0xffffffffu - ii[s]);
        }
        __syncthreads();
    };
    auto collect = [&](int64_t tie_end) {
        if (threadIdx.x == 0) {
            sh.count = 0;
            sh.bin_count = 0;
        }
        __syncthreads();
        for (int64_t e0 = 0; e0 < a.vocab; e0 += kBatch) {
            float v[kVpt];
            load_vals<DT, VEC>(row, e0, a.vocab, v);
#pragma unroll
            for (int vi = 0; vi < kVpt; ++vi) {
                const uint32_t key = sel_key(scale_logit(v[vi], temp, unit_temp));
                const int64_t e = val_index<DT>(e0, vi);
                if (key == 0u || key < theta_key || (key == theta_key && e >= tie_end)) continue;
                const int p = atomicAdd(&sh.count, 1);
                if (key > theta_key) atomicAdd(&sh.bin_count, 1);
                if (p < kPairCap)
                    pairs[p] = (static_cast<uint64_t>(key) << 32) | (0xffffffffu - static_cast<uint32_t>(e));
            }
        }
        __syncthreads();
    };
    if (source == kKeptInRow) {
        collect(a.vocab);
    } else {
        collect_from_lists();
    }
    int n = sh.count;
    if (n > kPairCap) {
        // Only ties at theta make that many: the values above it are fewer than the rank. The candidates are
        // those values and the first ties in index order.
        const int need = max(C - sh.bin_count, 0);
        const int64_t tie_end = nth_tie_end<DT, VEC>(a, row, temp, unit_temp, theta_key, need, sh);
        collect(tie_end);
        n = sh.count;
    }
    block_sort_desc_u64(pairs, n);
    markov_emit(pairs, min(n, C), C, a.noise + t * a.noise_stride, a.cand_ids + t * a.cand_stride,
                a.cand_probs + t * a.cand_stride, a.draws + t * a.draws_stride, sh);
}

// ---------------------------------------------------------------- Markov draw split over segments of the row
// With one workgroup per sequence a batch of 64 leaves three quarters of the chip idle, so the split draw cuts each
// row into segments of at most kSegKeys values, one workgroup each (8 at V = 151,936: 512 workgroups), in one
// launch (markov_draw_kernel). Each workgroup keeps its segment's keys in registers, 40 per thread (the Markov
// bias added and rounded to the logits' dtype, the temperature applied), and writes its keys at or above its own
// rank-th largest (rank = the row's top-k window; ties included, at most n_cand) as (key, index) pairs in (value
// descending, index ascending) order, with their count: a first bound from ballots over the lanes' largest keys
// leaves a short list of the keys at or above it, ranked exactly by comparing every pair with every other; a list
// past kShortCap (massive ties) takes range histograms instead. The row's candidates that can be kept are at or
// above the row's rank-th largest, which is at least every segment's, so they are all in the union of the
// segments' pairs. The pairs go to the coherence point, each segment counts itself on the row's counter, and the
// row's last segment to finish merges the lists and finishes as markov_tail does: the top-k threshold and the
// nucleus over the candidates (the same functions as probs_from_logits), Z, the race and the outputs.

constexpr int kSegKeys = 19456;          // values of one segment (at most 40 per thread, kept in registers)
constexpr int kSplitMaxCand = 512;       // candidates of the split draw (one per thread of the merging workgroup)
constexpr int kShortCap = 1024;          // a segment's short list, ranked pair by pair (past it: histograms)

struct MarkovSplitArgs {
    const void* logits;
    int64_t row_stride;
    const void* bias;            // [batch, vocab] in the logits' dtype, or null
    int64_t bias_stride;
    int64_t batch;
    int64_t vocab;
    const float* temps;
    const int64_t* top_k;
    const float* top_p;
    int max_top_k;
    int has_top_p;
    int n_cand;
    int seg_len;                 // a multiple of 8
    int n_seg;
    uint64_t* pairs;             // [batch, n_seg, n_cand], written and read at the coherence point
    int* seg_counts;             // [batch, n_seg] pairs each segment wrote (a prefix of its n_cand slots)
    int* counters;               // [batch] segments of the row finished; zero between calls
    const float* noise;
    int64_t noise_stride;
    int32_t* cand_ids;
    float* cand_probs;
    int64_t cand_stride;
    int64_t* draws;
    int64_t draws_stride;
};

template <int DT>
__device__ __forceinline__ float round_to_dtype(float x) {
    if constexpr (DT == NVS_DTYPE_F32) {
        return x;
    } else if constexpr (DT == NVS_DTYPE_BF16) {
        return static_cast<float>(static_cast<__bf16>(x));   // round to nearest even (one conversion on gfx950)
    } else {
        return __half2float(__float2half_rn(x));
    }
}

// Element `hi` (0: low half) of a 32-bit word holding two 16-bit values of the dtype.
template <int DT>
__device__ __forceinline__ float half_of(uint32_t w, int hi) {
    const uint16_t bits = static_cast<uint16_t>(hi ? (w >> 16) : (w & 0xffffu));
    if constexpr (DT == NVS_DTYPE_BF16) {
        return nvs::bf16_bits_to_float(bits);
    } else {
        return nvs::f16_bits_to_float(bits);
    }
}

// How many of the first n pairs of buf (LDS, read by every lane at once) are greater than x: eight loads in flight
// at a time rather than one round trip per pair.
__device__ __forceinline__ int count_above(const uint64_t* buf, int n, uint64_t x) {
    int above = 0;
    int j = 0;
    for (; j + 8 <= n; j += 8) {
        uint64_t v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = buf[j + u];
#pragma unroll
        for (int u = 0; u < 8; ++u) above += (v[u] > x) ? 1 : 0;
    }
    for (; j < n; ++j) above += (buf[j] > x) ? 1 : 0;
    return above;
}

// The merge of a row's segment lists by the row's last segment to finish (markov_draw_kernel). Each list (sorted,
// value descending, index ascending) and its count are read at the coherence point, all loads issued before any
// is used. When the lists hold at most one pair per thread (the usual case: about the window's size per segment),
// every pair is ranked against all the others at once; otherwise a tree of pairwise merges keeps the top n_cand of
// each pair of lists until one is left. Every pair is distinct (one index each). Then the top-k threshold and the
// nucleus over the candidates, Z, the race and the outputs, as markov_tail does: by wave 0 alone when the
// candidates fit two per lane and the window 64, else by the workgroup.
// noise_c and noise_c64 (the noise of candidates threadIdx.x and threadIdx.x + 64; C <= kSelThreads), tk and top_p
// were loaded before the row's count.
__device__ void markov_merge_row(const MarkovSplitArgs& a, int64_t b, float noise_c, float noise_c64, int64_t tk,
                                 float top_p, SelShared& sh) {
    uint64_t* pairs = pair_buf(sh);
    const int C = a.n_cand;
    const int total = a.n_seg * C;
    const uint64_t* src = a.pairs + b * total;
    uint64_t* all = pairs + kPairCap / 2;
    const int lane = lane_id();
    // every load issued before any is used: one round trip to the coherence point (total <= kPairCap / 2 pairs,
    // n_seg <= 64 counts, one per lane of every wave)
    constexpr int kPer = kPairCap / 2 / kSelThreads;
    const int rounds = (total + kSelThreads - 1) / kSelThreads;   // the rounds of slots that exist (uniform)
    uint64_t got[kPer];
#pragma unroll
    for (int r = 0; r < kPer; ++r) {
        got[r] = 0ull;
        if (r < rounds) {
            const int i = min(static_cast<int>(threadIdx.x) + r * kSelThreads, total - 1);
            got[r] = __hip_atomic_load(src + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    const int cnt_raw = __hip_atomic_load(a.seg_counts + b * a.n_seg + min(lane, a.n_seg - 1), __ATOMIC_RELAXED,
                                          __HIP_MEMORY_SCOPE_AGENT);
    const int cnt = lane < a.n_seg ? min(max(cnt_raw, 0), C) : 0;
    const int cincl = wave_scan_incl_dpp(cnt);
    const int n_all = __shfl(cincl, 63);   // pairs in all the lists
    int real = min(C, n_all);
    if (n_all <= kSelThreads) {
        // The lists one after another (list s from the sum of the counts before it). Then every pair's rank: its
        // place in its own list plus, in each other list, the number of pairs above it, by binary searches that
        // advance eight lists at a time (one LDS round trip per halving for all eight).
#pragma unroll
        for (int r = 0; r < kPer; ++r) {
            if (r >= rounds) break;
            const int e = static_cast<int>(threadIdx.x) + r * kSelThreads;
            const int li = e / C;
            const int i = e - li * C;
            const int c_li = __shfl(cnt, min(li, 63));
            const int off = __shfl(cincl, min(li, 63)) - c_li;
            if (e < total && i < c_li) all[off + i] = got[r];
        }
        int longest = cnt;
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) longest = max(longest, __shfl_xor(longest, o));
        __syncthreads();
        const int t = static_cast<int>(threadIdx.x);
        int own = 0;   // the list holding pair t: the number of lists that end at or before it
        for (int l = 0; l < a.n_seg; ++l) own += (__builtin_amdgcn_readlane(cincl, l) <= t) ? 1 : 0;
        const int own_start = __shfl(cincl, min(own, 63)) - __shfl(cnt, min(own, 63));
        if (t < n_all) {
            const uint64_t x = all[t];
            int above = t - own_start;   // its place in its own list
            // The count of a list's pairs above x (a prefix: the list is descending) by binary lifting: steps top,
            // top / 2, ..., 1, where top is the largest power of two not above the longest list, add up to any
            // count. A step is taken when the pair it lands on is inside the list and above x; the pairs it reads
            // past a list stay inside the pair space (at most n_all + 2 * longest < kPairCap / 2) and are unused.
            int top = 1;
            while (2 * top <= longest) top *= 2;
            for (int g0 = 0; g0 < a.n_seg; g0 += 8) {
                int pos[8], lim[8], base[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    const int l = min(g0 + u, a.n_seg - 1);
                    const int c_l = __builtin_amdgcn_readlane(cnt, l);
                    base[u] = __builtin_amdgcn_readlane(cincl, l) - c_l;
                    pos[u] = 0;
                    lim[u] = (g0 + u < a.n_seg && g0 + u != own) ? c_l : 0;
                }
                for (int step = top; step > 0; step >>= 1) {
                    uint64_t v[8];
#pragma unroll
                    for (int u = 0; u < 8; ++u) v[u] = all[base[u] + pos[u] + step - 1];   // every read, then the tests
#pragma unroll
                    for (int u = 0; u < 8; ++u) {
                        const bool take = (pos[u] + step - 1 < lim[u]) & (v[u] > x);
                        pos[u] += take ? step : 0;
                    }
                }
#pragma unroll
                for (int u = 0; u < 8; ++u) above += pos[u];
            }
            if (above < C) pairs[above] = x;
        }
        __syncthreads();
    } else {
        // the lists at their slots, zero past each count (zeros sort below every pair)
#pragma unroll
        for (int r = 0; r < kPer; ++r) {
            if (r >= rounds) break;
            const int e = static_cast<int>(threadIdx.x) + r * kSelThreads;
            const int li = e / C;
            const int i = e - li * C;
            const int c_li = __shfl(cnt, min(li, 63));
            if (e < total) all[e] = (i < c_li) ? got[r] : 0ull;
        }
        __syncthreads();
        // A tree of pairwise merges, each keeping the top C of its two lists: an element's rank in the merge is
        // its place in its own list plus the number of the other list's pairs above it (a branch-free binary
        // search). The nonzero pairs of two lists fill the first ranks, their zeros every rank after them, so every
        // slot of the output is written. Lists 2m and 2m+1 merge into list m of the other half of the pair space;
        // a last list without a mate is copied.
        uint64_t* cur = all;
        uint64_t* nxt = pairs;
        for (int n_lists = a.n_seg; n_lists > 1; n_lists = (n_lists + 1) / 2) {
            for (int e = threadIdx.x; e < n_lists * C; e += kSelThreads) {
                const int li = e / C;
                const int i = e - li * C;
                const uint64_t x = cur[e];
                const int mate = li ^ 1;
                int above = 0;
                if (mate < n_lists) {
                    const uint64_t* other = cur + mate * C;
                    int lo = 0, hi = C;
                    for (int len = C; len > 0; len >>= 1) {   // floor(log2 C) + 1 halvings empty the interval
                        const int mid = (lo + hi) >> 1;
                        const bool open = lo < hi;
                        const bool gt = other[min(mid, C - 1)] > x;
                        lo = (open && gt) ? mid + 1 : lo;
                        hi = (open && !gt) ? mid : hi;
                    }
                    above = lo;
                }
                const int rank = i + above;
                if (rank < C) nxt[(li >> 1) * C + rank] = x;
            }
            __syncthreads();
            uint64_t* t = cur;
            cur = nxt;
            nxt = t;
        }
        if (cur != pairs) {   // the top C of the union into the lower half (an odd number of levels leaves it above)
            for (int i = threadIdx.x; i < C; i += kSelThreads) pairs[i] = cur[i];
            __syncthreads();
        }
    }
    const int K = static_cast<int>(min(static_cast<int64_t>(a.max_top_k), a.vocab));
    int rank = static_cast<int>(min(tk > 0 ? tk : static_cast<int64_t>(K), static_cast<int64_t>(K)));
    rank = min(rank, real);
    if (C <= 128 && rank <= 64) {
        // Wave 0 alone, two candidates per lane (c = lane, lane + 64), with the workgroup path's arithmetic in the
        // same order (Z: the sum over the first 64 candidates, then over the next 64), so the results are the same.
        if (threadIdx.x >= 64) return;
        const uint64_t p0 = lane < real ? pairs[lane] : 0ull;
        const uint64_t p1 = lane + 64 < real ? pairs[lane + 64] : 0ull;
        const uint32_t k0 = static_cast<uint32_t>(p0 >> 32);
        const uint32_t k1 = static_cast<uint32_t>(p1 >> 32);
        uint32_t theta_key = 0xffffffffu;   // no value: nothing kept
        if (rank > 0) {
            const uint32_t thr_key = static_cast<uint32_t>(pairs[rank - 1] >> 32);
            float theta = nvs::key_float(thr_key);
            if (a.has_top_p) theta = wave_top_p_threshold64(lane < rank ? k0 : 0u, rank, K, top_p, theta);
            theta_key = nvs::float_key(theta);
        }
        // the kept candidates form a prefix of the sorted pairs
        const int kept = __popcll(__ballot(lane < real && k0 >= theta_key)) +
                         __popcll(__ballot(lane + 64 < real && k1 >= theta_key));
        const float m = kept > 0 ? nvs::key_float(static_cast<uint32_t>(__shfl(static_cast<int>(k0), 0))) : 0.f;
        const float e0 = lane < kept ? expf(nvs::key_float(k0) - m) : 0.f;
        const float e1 = lane + 64 < kept ? expf(nvs::key_float(k1) - m) : 0.f;
        const float z = wave_sum(e0) + wave_sum(e1);
        uint64_t best = 0;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int c = lane + 64 * h;
            if (c >= C) continue;
            const uint64_t pr = h ? p1 : p0;
            float p = 0.f;
            int32_t id = -1;
            if (c < kept) {
                p = expf(nvs::key_float(static_cast<uint32_t>(pr >> 32)) - m) / z;
                id = static_cast<int32_t>(0xffffffffu - static_cast<uint32_t>(pr));
            }
            a.cand_ids[b * a.cand_stride + c] = id;
            a.cand_probs[b * a.cand_stride + c] = p;
            const float score = p / (h ? noise_c64 : noise_c);
            const uint64_t k64 = (static_cast<uint64_t>(nvs::float_key(score)) << 32) |
                                 static_cast<uint64_t>(0xffffffffu - static_cast<uint32_t>(c));
            best = best > k64 ? best : k64;
        }
        best = wave_max_u64(best);
        if (lane == 0) {
            const float score = nvs::key_float(static_cast<uint32_t>(best >> 32));
            const int win = (score > 0.f) ? static_cast<int>(0xffffffffu - static_cast<uint32_t>(best)) : 0;
            a.draws[b * a.draws_stride] =
                win < kept ? static_cast<int64_t>(0xffffffffu - static_cast<uint32_t>(pairs[win])) : int64_t{0};
        }
        return;
    }
    uint32_t theta_key = 0xffffffffu;   // no value: nothing kept
    if (rank > 0) {
        const uint32_t thr_key = static_cast<uint32_t>(pairs[rank - 1] >> 32);
        float theta = nvs::key_float(thr_key);
        if (a.has_top_p) {
            for (int i = threadIdx.x; i < rank; i += kSelThreads) sh.sortbuf[i] = static_cast<uint32_t>(pairs[i] >> 32);
            __syncthreads();
            theta = top_p_threshold(sh, rank, K, top_p, theta);
        }
        theta_key = nvs::float_key(theta);
    }
    // the kept candidates form a prefix of the sorted pairs
    int kept = 0;
    for (int c = threadIdx.x; c < real; c += kSelThreads) kept += (static_cast<uint32_t>(pairs[c] >> 32) >= theta_key) ? 1 : 0;
    kept = static_cast<int>(block_sum(static_cast<float>(kept), sh));
    // probabilities exp(s - m) / Z over the kept candidates, the race argmax_c p_c / noise_c (first rank on ties,
    // rank 0 when every score is zero), the candidate row and the drawn token (markov_emit, one candidate per thread)
    const int c = threadIdx.x;
    const float m = kept > 0 ? nvs::key_float(static_cast<uint32_t>(pairs[0] >> 32)) : 0.f;
    float z = (c < kept) ? expf(nvs::key_float(static_cast<uint32_t>(pairs[c] >> 32)) - m) : 0.f;
    z = block_sum(z, sh);
    uint64_t best = 0;
    if (c < C) {
        float p = 0.f;
        int32_t id = -1;
        if (c < kept) {
            const uint64_t pr = pairs[c];
            p = expf(nvs::key_float(static_cast<uint32_t>(pr >> 32)) - m) / z;
            id = static_cast<int32_t>(0xffffffffu - static_cast<uint32_t>(pr));
        }
        a.cand_ids[b * a.cand_stride + c] = id;
        a.cand_probs[b * a.cand_stride + c] = p;
        const float score = p / noise_c;
        best = (static_cast<uint64_t>(nvs::float_key(score)) << 32) |
               static_cast<uint64_t>(0xffffffffu - static_cast<uint32_t>(c));
    }
    best = block_max_u64(best, sh);
    if (threadIdx.x == 0) {
        const float score = nvs::key_float(static_cast<uint32_t>(best >> 32));
        const int win = (score > 0.f) ? static_cast<int>(0xffffffffu - static_cast<uint32_t>(best)) : 0;
        a.draws[b * a.draws_stride] =
            win < kept ? static_cast<int64_t>(0xffffffffu - static_cast<uint32_t>(pairs[win])) : int64_t{0};
    }
}

template <int DT, bool VEC, bool BIAS>
__global__ __launch_bounds__(kSelThreads, 4) void markov_draw_kernel(MarkovSplitArgs a) {
#pragma clang fp contract(off)
    // One SelShared, its members reused phase by phase: the segment's selection (histogram bins, bounds, the short
    // list in the pair space), then, in the row's last segment, the merge (pair space, sort buffer, reductions).
    __shared__ SelShared sh;
    uint32_t* hist = sh.hist;
    int& n_gt = sh.bin_count;
    uint32_t& pick_bin = sh.sel_digit;
    uint32_t& pick_rem = sh.sel_remaining;
    uint64_t* seg_pairs = reinterpret_cast<uint64_t*>(sh.sortbuf);   // the histogram path's want pairs, unsorted
    uint32_t* wbound = sh.wlo;
    uint32_t* whi = sh.wmax;
    uint32_t& seg_theta = sh.sel_greater;   // the segment's want-th largest key
    uint32_t& seg_count = sh.sel_equal;     // pairs the segment writes
    constexpr int W = piece_elems<DT>();
    const int seg = blockIdx.x;
    const int64_t b = blockIdx.y;
    const int64_t e_lo = static_cast<int64_t>(seg) * a.seg_len;
    const int n = static_cast<int>(min(static_cast<int64_t>(a.seg_len), a.vocab - e_lo));
    const float temp = a.temps[b];
    const bool unit_temp = (temp == 1.f);
    const int64_t row_tk = a.top_k[b];
    // What the merge needs besides the lists, requested first (before the segment's keys, which then cannot delay
    // them): used only by the row's last segment.
    const int tid = static_cast<int>(threadIdx.x);
    const float noise_c = tid < a.n_cand ? a.noise[b * a.noise_stride + tid] : 1.f;
    const float noise_c64 = tid + 64 < a.n_cand ? a.noise[b * a.noise_stride + tid + 64] : 1.f;
    const float row_top_p = a.has_top_p ? a.top_p[b] : 1.f;
    const int es = nvs::dtype_size(DT);
    const char* row = static_cast<const char*>(a.logits) + (b * a.row_stride + e_lo) * es;
    const char* brow = BIAS ? static_cast<const char*>(a.bias) + (b * a.bias_stride + e_lo) * es : nullptr;
    // keys of the segment: s = dtype(logit + bias) / temperature (the reference's row_logits, then
    // probs_from_logits' division); NaN maps to key 0, below every value
    const int pieces = (n + W - 1) / W;
    // every piece of this thread requested before any is used (clamped into the segment, no branch: a load behind
    // a branch is sunk to its use and the requests would go out one round trip at a time)
    constexpr int kMaxPc = (kSegKeys / W + kSelThreads - 1) / kSelThreads;
    int (*tie_part)[kSelWaves] = reinterpret_cast<int (*)[kSelWaves]>(&sh.whist[0][0]);
    static_assert(kMaxPc * kSelWaves <= kSelWaves * 256, "the tie counts must fit the refinement histograms");
    u32x4 raw[kMaxPc];
    u32x4 braw[BIAS ? kMaxPc : 1];
#pragma unroll
    for (int j = 0; j < kMaxPc; ++j) {
        const int pc = min(static_cast<int>(threadIdx.x) + j * kSelThreads, pieces - 1);
        if constexpr (VEC) {
            raw[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(row) + pc);
            if constexpr (BIAS) braw[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(brow) + pc);
        } else {
            // element loads, packed like the 16-byte pieces (clamped indices)
            uint32_t w4[4] = {0u, 0u, 0u, 0u}, b4[4] = {0u, 0u, 0u, 0u};
#pragma unroll
            for (int c = 0; c < W; ++c) {
                const int i = min(pc * W + c, n - 1);
                if constexpr (DT == NVS_DTYPE_F32) {
                    w4[c] = reinterpret_cast<const uint32_t*>(row)[i];
                    if constexpr (BIAS) b4[c] = reinterpret_cast<const uint32_t*>(brow)[i];
                } else {
                    const uint32_t h = reinterpret_cast<const uint16_t*>(row)[i];
                    w4[c >> 1] |= (c & 1) ? (h << 16) : h;
                    if constexpr (BIAS) {
                        const uint32_t hb = reinterpret_cast<const uint16_t*>(brow)[i];
                        b4[c >> 1] |= (c & 1) ? (hb << 16) : hb;
                    }
                }
            }
            raw[j] = u32x4{w4[0], w4[1], w4[2], w4[3]};
            if constexpr (BIAS) braw[j] = u32x4{b4[0], b4[1], b4[2], b4[3]};
        }
    }
    uint32_t tmax = 0u;   // this thread's largest key
    // The thread's keys stay in registers. Register slot q holds element (threadIdx.x + (q / W) * kSelThreads) *
    // W + q % W, so index order is (q / W, thread, q % W); the valid slots are a prefix, q < qlim. Slots past the
    // segment hold key 0, which leaves tmax as it is; every later use of a slot also checks q < qlim.
    uint32_t kr[kMaxPc * W];
    int lim[kMaxPc];   // valid elements of each of the thread's pieces (0 past the segment)
    int qlim = 0;
#pragma unroll
    for (int j = 0; j < kMaxPc; ++j) {
        const int pc = static_cast<int>(threadIdx.x) + j * kSelThreads;
        lim[j] = max(0, min(W, n - pc * W));
        if (lim[j] > 0) qlim = j * W + lim[j];
    }
    // The temperature and the segment's shape are the same for the whole workgroup: one branch picks the loop,
    // rather than a select per key that would run the division for unit temperatures too.
    auto convert = [&](auto unit_c, auto whole_c) {
        constexpr bool kUnit = decltype(unit_c)::value;     // temperature 1: no division
        constexpr bool kWhole = decltype(whole_c)::value;   // every piece of the segment whole (n % W == 0)
#pragma unroll
        for (int j = 0; j < kMaxPc; ++j) {
            const uint32_t w4[4] = {raw[j].x, raw[j].y, raw[j].z, raw[j].w};
            float v[W];
            float bv[W];
            if constexpr (DT == NVS_DTYPE_F32) {
#pragma unroll
                for (int c = 0; c < 4; ++c) v[c] = __uint_as_float(w4[c]);
            } else {
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    v[2 * c] = half_of<DT>(w4[c], 0);
                    v[2 * c + 1] = half_of<DT>(w4[c], 1);
                }
            }
            if constexpr (BIAS) {
                const uint32_t b4[4] = {braw[j].x, braw[j].y, braw[j].z, braw[j].w};
                if constexpr (DT == NVS_DTYPE_F32) {
#pragma unroll
                    for (int c = 0; c < 4; ++c) bv[c] = __uint_as_float(b4[c]);
                } else {
#pragma unroll
                    for (int c = 0; c < 4; ++c) {
                        bv[2 * c] = half_of<DT>(b4[c], 0);
                        bv[2 * c + 1] = half_of<DT>(b4[c], 1);
                    }
                }
            }
            const bool piece_in = lim[j] > 0;
#pragma unroll
            for (int c = 0; c < W; ++c) {
                float x = v[c];
                if constexpr (BIAS) x = round_to_dtype<DT>(x + bv[c]);
                if constexpr (!kUnit) x = x / temp;
                const bool in = kWhole ? piece_in : (c < lim[j]);
                const uint32_t key = in ? sel_key(x) : 0u;
                kr[j * W + c] = key;
                tmax = max(tmax, key);
            }
        }
    };
    const bool whole = (n % W) == 0;
    if (unit_temp) {
        if (whole) convert(std::true_type{}, std::true_type{});
        else convert(std::true_type{}, std::false_type{});
    } else {
        if (whole) convert(std::false_type{}, std::true_type{});
        else convert(std::false_type{}, std::false_type{});
    }
    __syncthreads();
    // The segment's want-th largest key, want = the row's top-k window (a row without top-k: max_top_k) or the
    // segment's length. A lower bound first: each wave's ceil(want / 8)-th largest lane maximum, rounded down to a
    // multiple of 2^16 (one ballot for each of the upper 16 bits: exact for 16-bit logits, whose keys carry no
    // more), the smallest over the waves; every wave has that many lanes holding a key at or above it, so at least
    // `want` keys are.
    const int K = static_cast<int>(min(static_cast<int64_t>(a.max_top_k), a.vocab));
    const int want = static_cast<int>(min(min(row_tk > 0 ? row_tk : static_cast<int64_t>(K), static_cast<int64_t>(K)),
                                          static_cast<int64_t>(n)));
    const int rw = (want + kSelWaves - 1) / kSelWaves;   // <= 64: K <= n_cand <= kSplitMaxCand
    uint32_t wb = 0u;
#pragma unroll
    for (int bit = 31; bit >= 16; --bit) {
        const uint32_t cand = wb | (1u << bit);
        if (static_cast<int>(__popcll(__ballot(tmax >= cand))) >= rw) wb = cand;
    }
    const uint32_t wmaxk = wave_max_u32(tmax);
    if (lane_id() == 0) {
        wbound[threadIdx.x >> 6] = wb;
        whi[threadIdx.x >> 6] = wmaxk;
    }
    if (threadIdx.x == 0) {
        sh.count = 0;
        seg_count = 0u;
    }
    __syncthreads();
    uint32_t lo = 0xffffffffu, hi = 0u;
    for (int w = 0; w < kSelWaves; ++w) {
        lo = min(lo, wbound[w]);
        hi = max(hi, whi[w]);
    }
    uint64_t* out = a.pairs + (b * a.n_seg + seg) * a.n_cand;
    // the segment's pairs go to the coherence point, where the row's merging workgroup (any XCD) reads them
    auto put = [&](int idx, uint64_t v) { __hip_atomic_store(out + idx, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); };
    // The short list: every key at or above the bound (at least want of them), appended wave by wave as
    // (key, index) pairs to the pair space: each lane's count, one prefix over the wave and one reservation per
    // wave, then the lane's keys in order.
    uint64_t* list = pair_buf(sh);
    // With a bound above key 0 the slots past the segment (key 0) fail the test by themselves; only a bound of 0
    // needs q < qlim as well.
    auto short_list = [&](auto all_c) {
        constexpr bool kCheckSlot = decltype(all_c)::value;
        auto passes = [&](int q) { return (!kCheckSlot || q < qlim) && kr[q] >= lo; };
        int mine = 0;
#pragma unroll
        for (int q = 0; q < kMaxPc * W; ++q) mine += passes(q) ? 1 : 0;
        const int incl = wave_scan_incl_dpp(mine);
        int base = 0;
        if (lane_id() == 63 && incl > 0) base = atomicAdd(&sh.count, incl);
        int p = __builtin_amdgcn_readlane(base, 63) + incl - mine;
#pragma unroll
        for (int q = 0; q < kMaxPc * W; ++q) {
            if (passes(q)) {
                if (p < kShortCap) {
                    const int i = (static_cast<int>(threadIdx.x) + (q / W) * kSelThreads) * W + q % W;
                    list[p] = (static_cast<uint64_t>(kr[q]) << 32) | (0xffffffffu - static_cast<uint32_t>(e_lo + i));
                }
                ++p;
            }
        }
    };
    if (lo > 0u) short_list(std::false_type{});
    else short_list(std::true_type{});
    __syncthreads();
    const int nl = sh.count;
    if (nl <= kShortCap) {
        // Every pair's rank in the list (all pairs differ: one index each). The pair ranked want - 1 holds the
        // segment's want-th largest key; every pair at or above that key (the ties after it included) goes to its
        // rank, up to n_cand of them.
        uint64_t pv[kShortCap / kSelThreads];
        int pa[kShortCap / kSelThreads];
#pragma unroll
        for (int r = 0; r < kShortCap / kSelThreads; ++r) {
            const int p = static_cast<int>(threadIdx.x) + r * kSelThreads;
            pv[r] = 0ull;
            pa[r] = kShortCap;
            if (p < nl) {
                const uint64_t v = list[p];
                const int above = count_above(list, nl, v);
                pv[r] = v;
                pa[r] = above;
                if (above == want - 1) seg_theta = static_cast<uint32_t>(v >> 32);
            }
        }
        __syncthreads();
        const uint32_t th = seg_theta;
        uint32_t mine = 0u;
#pragma unroll
        for (int r = 0; r < kShortCap / kSelThreads; ++r) {
            if (pa[r] < a.n_cand && static_cast<uint32_t>(pv[r] >> 32) >= th) {
                put(pa[r], pv[r]);
                ++mine;
            }
        }
        if (mine > 0u) atomicAdd(&seg_count, mine);
    } else {
    // Massive ties at the bound: range histograms find the want-th largest key, the keys above it are taken, then
    // the ties at it in index order, up to n_cand pairs in all.
    uint32_t span = hi - lo;
    uint32_t rank = static_cast<uint32_t>(want);
    for (int pass = 0; pass < 5; ++pass) {
        const int shift = span < 256u ? 0 : 24 - __clz(span);   // (span >> shift) < 256
        if (threadIdx.x < 256) hist[threadIdx.x] = 0u;
        __syncthreads();
#pragma unroll
        for (int q = 0; q < kMaxPc * W; ++q) {
            const uint32_t d = kr[q] - lo;   // wraps for keys below lo, which then exceed span
            if (q < qlim && kr[q] >= lo && d <= span) atomicAdd(&hist[d >> shift], 1u);
        }
        __syncthreads();
        if (threadIdx.x < 64) {
            uint32_t bin, rem;
            wave_pick_bin(hist, rank, bin, rem);
            if (threadIdx.x == 0) {
                pick_bin = bin;
                pick_rem = rem;
            }
        }
        __syncthreads();
        lo += pick_bin << shift;
        rank = pick_rem;
        if (shift == 0) break;
        span = (1u << shift) - 1u;
    }
    const uint32_t t_key = lo;
    // The keys above the threshold (fewer than want) in any order, then the first n_cand - n_gt ties in index
    // order. Ties of each register group are counted per thread, and one workgroup prefix over all groups at once
    // gives every tie its rank.
    if (threadIdx.x == 0) n_gt = 0;
    int cnt[kMaxPc];
#pragma unroll
    for (int j = 0; j < kMaxPc; ++j) {
        cnt[j] = 0;
#pragma unroll
        for (int c = 0; c < W; ++c) cnt[j] += (j * W + c < qlim && kr[j * W + c] == t_key) ? 1 : 0;
    }
    int incl[kMaxPc];
#pragma unroll
    for (int j = 0; j < kMaxPc; ++j) incl[j] = wave_scan_incl_dpp(cnt[j]);
    __syncthreads();
    if (lane_id() == 63) {
#pragma unroll
        for (int j = 0; j < kMaxPc; ++j) tie_part[j][threadIdx.x >> 6] = incl[j];
    }
#pragma unroll
    for (int q = 0; q < kMaxPc * W; ++q) {
        const uint32_t k = kr[q];
        if (q < qlim && k > t_key) {
            const int i = (static_cast<int>(threadIdx.x) + (q / W) * kSelThreads) * W + q % W;
            seg_pairs[atomicAdd(&n_gt, 1)] = (static_cast<uint64_t>(k) << 32) |
                                             (0xffffffffu - static_cast<uint32_t>(e_lo + i));
        }
    }
    __syncthreads();
    const int gt = n_gt;
    const int need = a.n_cand - gt;
    const int wave = static_cast<int>(threadIdx.x >> 6);
    int base = 0;   // ties of earlier groups, every thread
#pragma unroll
    for (int j = 0; j < kMaxPc; ++j) {
        int before = 0, total_j = 0;
        for (int w = 0; w < kSelWaves; ++w) {
            const int c = tie_part[j][w];
            total_j += c;
            before += (w < wave) ? c : 0;
        }
        int r = base + before + incl[j] - cnt[j];   // rank of this thread's first tie of group j
#pragma unroll
        for (int c = 0; c < W; ++c) {
            const int q = j * W + c;
            if (q < qlim && kr[q] == t_key) {
                if (r < need) {
                    const int i = (static_cast<int>(threadIdx.x) + j * kSelThreads) * W + c;
                    seg_pairs[gt + r] = (static_cast<uint64_t>(t_key) << 32) |
                                        (0xffffffffu - static_cast<uint32_t>(e_lo + i));
                }
                ++r;
            }
        }
        base += total_j;
    }
    // the segment's pairs, sorted: each pair goes to its rank among them (all distinct)
    const int n_out = gt + min(base, need);
    __syncthreads();
    for (int p = threadIdx.x; p < n_out; p += kSelThreads) {
        const uint64_t v = seg_pairs[p];
        put(count_above(seg_pairs, n_out, v), v);
    }
    if (threadIdx.x == 0) seg_count = static_cast<uint32_t>(n_out);
    }

    // Count the segment on the row's counter once every wave's stores (and thread 0's count) have completed; the
    // row's last segment to count merges. Its loads are issued after its own count returned, at the coherence point.
    __syncthreads();
    if (threadIdx.x == 0)
        __hip_atomic_store(a.seg_counts + b * a.n_seg + seg, static_cast<int>(seg_count), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0)
    __syncthreads();
    if (threadIdx.x == 0) {
        const int before = __hip_atomic_fetch_add(a.counters + b, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        sh.last = (before == a.n_seg - 1) ? 1 : 0;
    }
    __syncthreads();
    if (!sh.last) return;
    if (threadIdx.x == 0) __hip_atomic_store(a.counters + b, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    markov_merge_row(a, b, noise_c, noise_c64, row_tk, row_top_p, sh);
}


// WIDE: instantiated for batches whose max_top_k exceeds the candidate lists (kMaxTopK); the others never carry
// the wide path's code.
template <int DT, int MODE, bool VEC, bool WIDE>
// At most 128 VGPRs (4 waves per SIMD): two 8-wave workgroups per CU, so the 512 positions of a verify batch
// run in one round on 256 CUs.
__global__ __launch_bounds__(kSelThreads, 4) void select_kernel(SelArgs a) {
    __shared__ SelShared sh;
    const int64_t t = blockIdx.x;
    if (threadIdx.x == 0) {
        sh.count = 0;
        sh.overflow = 0;
        sh.found = 0;
        sh.last = 0;
        sh.tau_key = 0u;
        sh.loc[0] = sh.loc[1] = sh.loc[3] = 0;
        sh.loc[2] = 1;
    }
    __syncthreads();
    int64_t prow;
    if constexpr (MODE == kModeAccept) {
        locate(a, t, sh);
        prow = sh.loc[0];
    } else {
        prow = t / a.pos_per_param;
    }
    const float temp = a.temps != nullptr ? a.temps[prow] : 1.f;
    const bool unit_temp = (temp == 1.f);
    const int64_t tk = a.top_k != nullptr ? a.top_k[prow] : 0;
    const float top_p = a.top_p != nullptr ? a.top_p[prow] : 1.f;
    const int K = static_cast<int>(min(static_cast<int64_t>(a.max_top_k), a.vocab));
    // A Markov draw, and an accept whose q comes as candidate rows, always truncate (every row of a candidate
    // batch has top-k); a row without top-k there is treated as top-k max_top_k.
    const bool truncating = K > 0 && (tk > 0 || MODE == kModeMarkov || (MODE == kModeAccept && a.q_ids != nullptr));
    const int rank = truncating ? static_cast<int>(min(tk > 0 ? tk : static_cast<int64_t>(K),
                                                       static_cast<int64_t>(K))) : 0;
    const char* row = static_cast<const char*>(a.logits) + t * a.row_stride * nvs::dtype_size(DT);

    // Fused accept: the accept test's inputs (draft token d, the logit at d, q at d, the uniform) do not depend on
    // the pass over the row, so every thread requests them (same addresses, clamped into range: no branch) before
    // the row streams, and they arrive while it does. dec_valid: this position verifies a draft inside the
    // vocabulary (an out-of-vocabulary draft is never accepted).
    bool dec_valid = false;
    float dec_x = 0.f, dec_q = 0.f, dec_u = 0.f;
    int64_t dec_slot = 0, dec_d = 0;
    if constexpr (MODE == kModeAccept) {
        const int64_t b = sh.loc[0], j = sh.loc[1], L = sh.loc[2];
        dec_slot = b * a.k + min(j, static_cast<int64_t>(a.k) - 1);
        dec_d = a.drafts[dec_slot];
        dec_valid = (j < L - 1) && (j < a.k) && (dec_d >= 0) && (dec_d < a.vocab);
    }
    auto load_decision = [&]() {
        if constexpr (MODE == kModeAccept) {
            const int64_t dc = min(max(dec_d, int64_t{0}), a.vocab - 1);
            dec_x = nvs::load_as_float<DT>(row, dc);
            dec_q = a.q_ids == nullptr ? a.q[dec_slot * a.vocab + dc] : 0.f;   // candidate rows: found later
            dec_u = a.uniforms[dec_slot];
        }
    };

    RowStats rs;
    rs.dense = !truncating;
    rs.theta = -INFINITY;
    bool record_done = false;   // the wave-0 epilogue already wrote this position's record
    int kept_source = kKeptInRow;   // where a Markov draw finds the kept values
    if (!truncating) {
        // online max / sum-exp over the whole row, one batch at a time: the batch's max rescales the running sum
        // once, then every value adds exp(s - m). NaN (and the padding past the row) adds nothing; -inf adds 0.
        // The pass is bound by its arithmetic: the division by the temperature and the mask of the last, partial
        // batch sit behind uniform branches (as selects they would be computed for every value).
        float m = -INFINITY, z = 0.f;
        const int nb = static_cast<int>((a.vocab + kBatch - 1) / kBatch);
        auto accum = [&](float (&v)[kVpt], int bi) {
            if (bi == nb - 1) {
                const int64_t e0 = static_cast<int64_t>(bi) * kBatch;
#pragma unroll
                for (int vi = 0; vi < kVpt; ++vi) v[vi] = val_index<DT>(e0, vi) < a.vocab ? v[vi] : NAN;
            }
            if (!unit_temp) {
#pragma unroll
                for (int vi = 0; vi < kVpt; ++vi) v[vi] = v[vi] / temp;
            }
            float bm = v[0];
#pragma unroll
            for (int vi = 1; vi < kVpt; ++vi) bm = fmaxf(bm, v[vi]);
            if (bm > m) {
                z = z * expf(m - bm);
                m = bm;
            }
            if (m == -INFINITY) return;
#pragma unroll
            for (int vi = 0; vi < kVpt; ++vi) z += (v[vi] == v[vi]) ? expf(v[vi] - m) : 0.f;
        };
        // three buffers in a ring (two with element loads): this pass is bound by its arithmetic, not its loads
        float ra[kVpt], rb[kVpt], rc[kVpt];
        load_vals<DT, VEC, false>(row, 0, a.vocab, ra);
        load_vals<DT, VEC, false>(row, kBatch, a.vocab, rb);
        if constexpr (VEC) load_vals<DT, VEC, false>(row, 2 * kBatch, a.vocab, rc);
        load_decision();
        if constexpr (VEC) {
            for (int bi = 0;;) {
                accum(ra, bi);
                load_vals<DT, VEC, false>(row, static_cast<int64_t>(bi + 3) * kBatch, a.vocab, ra);
                if (++bi >= nb) break;
                accum(rb, bi);
                load_vals<DT, VEC, false>(row, static_cast<int64_t>(bi + 3) * kBatch, a.vocab, rb);
                if (++bi >= nb) break;
                accum(rc, bi);
                load_vals<DT, VEC, false>(row, static_cast<int64_t>(bi + 3) * kBatch, a.vocab, rc);
                if (++bi >= nb) break;
            }
        } else {
            for (int bi = 0;;) {
                accum(ra, bi);
                if (++bi >= nb) break;
                load_vals<DT, VEC, false>(row, static_cast<int64_t>(bi + 1) * kBatch, a.vocab, ra);
                accum(rb, bi);
                if (++bi >= nb) break;
                load_vals<DT, VEC, false>(row, static_cast<int64_t>(bi + 1) * kBatch, a.vocab, rb);
            }
        }
        const uint32_t mk = block_max_u32(m == -INFINITY ? 0u : nvs::float_key(m), sh);
        const float mall = mk == 0u ? -INFINITY : nvs::key_float(mk);
        const float mu = (mall == -INFINITY) ? 0.f : mall;
        const float zz = (m == -INFINITY) ? 0.f : z * expf(m - mu);
        rs.z = block_sum(zz, sh);
        rs.m = mall;
    } else {
        // ---- one pass: every element >= tau, a lower bound of the K-th largest, joins a candidate list private
        // to its lane: kLaneCap slots, slot s of lane l of wave w at sh.ckey[w * kWaveSlots + s * 64 + l] (the
        // index at the same place in sh.cidx). tau starts from the first two batches (see below), a value with at
        // least K elements at or above it. After that the pass has no workgroup barrier and the append no
        // cross-lane step. When some lane of a wave has filled three quarters of its slots, the wave raises tau to
        // a bound of the K-th largest of its own lists (a lower bound of the row's too), drops what lies below and
        // publishes the bound to the other waves through one LDS word they read each batch. A lane whose list
        // still overflows sends the row to the exact path.
        const int wave = threadIdx.x >> 6;
        const int lane = lane_id();
        uint32_t* wkey = sh.ckey + wave * kWaveSlots;
        int32_t* widx = sh.cidx + wave * kWaveSlots;
        const int nb = static_cast<int>((a.vocab + kBatch - 1) / kBatch);
        uint32_t tau_key = 0xffffffffu;
        float tau = INFINITY;
        int lcnt = 0;           // this lane's list length
        uint32_t hmax = 0u;     // largest key this lane appended
        // the same on every lane of the wave. A window wider than the candidate lists (K > kMaxTopK, beyond the
        // first bound's reach) starts overflowed: the pass then only streams the row, and the exact path decides
        // every truncating row of the batch (the wide ones without any list, wide_row_stats)
        bool overflow = WIDE && K > kMaxTopK;
        // With a positive temperature the pass compares raw values: x / t rounds monotonically in x, so the K-th
        // largest scaled value is the K-th largest raw value divided by t, and the lists are scaled once at the end
        // of the pass instead of every value in it. Two adjacent raw values can divide to the same quotient, so the
        // raw bound is lowered by one unit in the last place: a value just below it whose quotient ties with the
        // bound's is listed too. A temperature that is not positive and finite scales every value in the pass.
        const bool raw_mode = !unit_temp && temp > 0.f && temp < INFINITY;
        const bool scale_in_pass = !unit_temp && !raw_mode;
        const uint32_t slack = raw_mode ? 1u : 0u;
        auto key_bound = [&](uint32_t k) { return k <= slack ? -INFINITY : nvs::key_float(k - slack); };

        // A tighter bound from this wave's lists: one 256-bin histogram of the listed keys at or above tau, the
        // bins spread over [tau, the wave's largest key]; the lower edge of the bin holding the wave's K-th largest
        // has at least K listed keys at or above it. Entries below the new bound leave the lists.
        auto refine = [&]() {
            if (wave_sum_i32(lcnt) < K) return;   // too few keys to bound the K-th largest
            const int max_cnt = static_cast<int>(wave_max_u32(static_cast<uint32_t>(lcnt)));
            const uint32_t whi = wave_max_u32(hmax);
            if (whi > tau_key) {
                uint32_t* hist = sh.whist[wave];
                const uint32_t range = whi - tau_key;
                const int sh_bits = range < 256u ? 0 : 24 - __clz(range);
#pragma unroll
                for (int i = 0; i < 4; ++i) hist[4 * lane + i] = 0u;
                compiler_fence_s();
                for (int s = 0; s < max_cnt; ++s) {
                    if (s < lcnt) {
                        const uint32_t k = wkey[s * 64 + lane];
                        if (k >= tau_key) atomicAdd(&hist[(k - tau_key) >> sh_bits], 1u);
                    }
                }
                compiler_fence_s();
                uint32_t b, r;
                wave_pick_bin(hist, static_cast<uint32_t>(K), b, r);
                compiler_fence_s();
                if (b < 256u && b > 0u) {
                    const uint32_t kb = tau_key + (b << sh_bits);
                    tau_key = kb;
                    tau = key_bound(kb);
                    atomicMax(&sh.tau_key, kb);
                }
            }
            // each lane compacts its own list in place (slot kept <= s: every read precedes the write over it)
            compiler_fence_s();
            int kept = 0;
            for (int s = 0; s < lcnt; ++s) {
                const uint32_t k = wkey[s * 64 + lane];
                const int32_t ix = widx[s * 64 + lane];
                if (k >= tau_key) {
                    wkey[kept * 64 + lane] = k;
                    widx[kept * 64 + lane] = ix;
                    ++kept;
                }
            }
            compiler_fence_s();
            lcnt = kept;
        };

        // Filter one batch. Most batches hold no element at or above tau in the whole wave: one max, one compare,
        // one ballot. Otherwise each lane with a passing value appends it to its own list.
        auto filter = [&](float (&sv)[kVpt], int bi) {   // may scale the buffer in place (it is reloaded next)
            const int64_t e0 = static_cast<int64_t>(bi) * kBatch;
            if (scale_in_pass) {
#pragma unroll
                for (int vi = 0; vi < kVpt; ++vi) sv[vi] = sv[vi] / temp;
            }
            if (e0 + kBatch > a.vocab) {   // the last, partial batch: elements past the row are NaN
#pragma unroll
                for (int vi = 0; vi < kVpt; ++vi) sv[vi] = val_index<DT>(e0, vi) < a.vocab ? sv[vi] : NAN;
            }
            const uint32_t shared_key = __hip_atomic_load(&sh.tau_key, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            // every path reads the whole buffer first, so its loads are complete before the buffer is reloaded
            float hi = sv[0];
#pragma unroll
            for (int vi = 1; vi < kVpt; ++vi) hi = fmaxf(hi, sv[vi]);
            if (overflow || __ballot(hi >= tau) == 0ull) return;
            if (shared_key > tau_key) {   // another wave raised the bound
                tau_key = shared_key;
                tau = key_bound(shared_key);
            }
            if (hi >= tau) {
#pragma unroll
                for (int vi = 0; vi < kVpt; ++vi) {
                    if (sv[vi] >= tau) {
                        const uint32_t key = nvs::float_key(sv[vi]);
                        // a full list overwrites its last slot; the overflow test below then sends the row to the
                        // exact path
                        const int s = min(lcnt, kLaneCap - 1);
                        wkey[s * 64 + lane] = key;
                        widx[s * 64 + lane] = static_cast<int32_t>(val_index<DT>(e0, vi));
                        hmax = max(hmax, key);
                        ++lcnt;
                    }
                }
            }
            if (__ballot(lcnt > kLaneCap * 3 / 4) == 0ull) return;
            if (__ballot(lcnt > kLaneCap) != 0ull) {
                overflow = true;   // the exact path re-reads the row
                return;
            }
            refine();
        };

        // Register buffers in a ring, unrolled so no values are copied: while one batch is filtered the next ones
        // are in flight. fp32 rows use two buffers (a pure read in this launch shape streams as fast with one or
        // two batches in flight per thread as with three, and the fused pass measured 0.5 us faster with two);
        // 16-bit rows, whose batches are half the bytes, use three (0.9 us faster than two on bf16 logits; four
        // need scratch). The loads are unconditional: a load guarded by a branch is sunk by the compiler to its
        // use, which leaves nothing in flight during the filter. Past the row every lane's address clamps to the
        // row's last piece (one cache line, never used).
        constexpr int kRing = (DT == NVS_DTYPE_F32 || !VEC) ? 2 : 3;
        float ra[kVpt], rb[kVpt], rc[kRing == 3 ? kVpt : 1];
        load_vals<DT, VEC, false>(row, 0, a.vocab, ra);
        load_vals<DT, VEC, false>(row, kBatch, a.vocab, rb);
        if constexpr (kRing == 3) load_vals<DT, VEC, false>(row, 2 * kBatch, a.vocab, rc);
        load_decision();   // after the draft token, behind the first batches
        {
            // The first bound: each lane's largest value over the first two batches, each wave's ceil(K/8)-th
            // largest lane maximum, the smallest of those over the 8 waves. Every wave has ceil(K/8) lanes holding
            // a value at or above it, so at least K elements of the row do.
            // The largest scaled value is the largest raw value divided by a positive temperature (division
            // rounds monotonically), the smallest one for a negative temperature.
            float mx = -INFINITY, mn = INFINITY;
#pragma unroll
            for (int vi = 0; vi < kVpt; ++vi) {
                const bool ina = val_index<DT>(0, vi) < a.vocab, inb = val_index<DT>(kBatch, vi) < a.vocab;
                mx = fmaxf(mx, fmaxf(ina ? ra[vi] : -INFINITY, inb ? rb[vi] : -INFINITY));
                mn = fminf(mn, fminf(ina ? ra[vi] : INFINITY, inb ? rb[vi] : INFINITY));
            }
            // A lane with nothing (or only -inf) counts as holding nothing: that can only lower the bound.
            const float ext = scale_in_pass ? scale_logit(temp < 0.f ? mn : mx, temp, unit_temp) : mx;
            const uint32_t tmax = (ext == -INFINITY || ext != ext) ? 0u : sel_key(ext);
            const int rw = (K + kSelWaves - 1) / kSelWaves;
            // the rw-th largest lane maximum, bit by bit from the top: the largest key with at least rw lanes at or
            // above it (one compare and one ballot per bit, no cross-lane data movement)
            uint32_t bound = 0u;
            if (rw <= 64) {
#pragma unroll
                for (int bit = 31; bit >= 0; --bit) {
                    const uint32_t cand = bound | (1u << bit);
                    if (static_cast<int>(__popcll(__ballot(tmax >= cand))) >= rw) bound = cand;
                }
            }
            if (lane == 0) sh.ured[wave] = bound;
            __syncthreads();
            uint32_t b = 0xffffffffu;
            for (int w = 0; w < kSelWaves; ++w) b = min(b, sh.ured[w]);
            tau_key = b;
            tau = key_bound(b);   // -inf for no bound; NaN never passes a >= test
        }
        if constexpr (VEC && kRing == 2) {
            // each buffer is reloaded with the batch two ahead as soon as it is filtered
            for (int bi = 0;;) {
                filter(ra, bi);
                load_vals<DT, VEC, false>(row, static_cast<int64_t>(bi + 2) * kBatch, a.vocab, ra);
                if (++bi >= nb) break;
                filter(rb, bi);
                load_vals<DT, VEC, false>(row, static_cast<int64_t>(bi + 2) * kBatch, a.vocab, rb);
                if (++bi >= nb) break;
            }
        } else if constexpr (VEC) {
            // the same with three buffers, each reloaded with the batch three ahead
            for (int bi = 0;;) {
                filter(ra, bi);
                load_vals<DT, VEC, false>(row, static_cast<int64_t>(bi + 3) * kBatch, a.vocab, ra);
                if (++bi >= nb) break;
                filter(rb, bi);
                load_vals<DT, VEC, false>(row, static_cast<int64_t>(bi + 3) * kBatch, a.vocab, rb);
                if (++bi >= nb) break;
                filter(rc, bi);
                load_vals<DT, VEC, false>(row, static_cast<int64_t>(bi + 3) * kBatch, a.vocab, rc);
                if (++bi >= nb) break;
            }
        } else {
            // element loads need an address per value: two buffers, one batch in flight, keep it in registers
            for (int bi = 0;;) {
                filter(ra, bi);
                if (++bi >= nb) break;
                load_vals<DT, VEC, false>(row, static_cast<int64_t>(bi + 1) * kBatch, a.vocab, ra);
                filter(rb, bi);
                if (++bi >= nb) break;
                load_vals<DT, VEC, false>(row, static_cast<int64_t>(bi + 1) * kBatch, a.vocab, rb);
            }
        }
        lcnt = min(lcnt, kLaneCap);   // past it only when the row goes to the exact path
        // The lane's list in registers, read in one LDS round trip (slots past lcnt are never used): the loops
        // below over the list would otherwise wait for one LDS read per slot.
        uint32_t lk[kLaneCap];
#pragma unroll
        for (int s = 0; s < kLaneCap; ++s) lk[s] = wkey[s * 64 + lane];
        if (raw_mode) {
            // the lists, the bound and the largest key move to scaled values: one division per listed value
#pragma unroll
            for (int s = 0; s < kLaneCap; ++s) {
                if (s < lcnt) {
                    lk[s] = nvs::float_key(nvs::key_float(lk[s]) / temp);
                    wkey[s * 64 + lane] = lk[s];
                }
            }
            tau_key = tau_key == 0u ? 0u : nvs::float_key(nvs::key_float(tau_key) / temp);
            hmax = hmax == 0u ? 0u : nvs::float_key(nvs::key_float(hmax) / temp);
        }
        const uint32_t wave_hi = wave_max_u32(hmax);
        const int wave_total = wave_sum_i32(lcnt);
        if (lane == 0) {
            sh.wcount[wave] = wave_total;
            if (overflow) sh.overflow = 1;
            sh.wlo[wave] = tau_key;
            sh.wmax[wave] = wave_hi;
        }
        if (threadIdx.x < 256) sh.hist[threadIdx.x] = 0u;
        if (threadIdx.x == 0) {
            sh.count = 0;
            sh.bin_count = 0;
        }
        __syncthreads();
        int listed = 0;
        for (int w = 0; w < kSelWaves; ++w) listed += sh.wcount[w];
        // fewer listed keys than the rank (NaN logits never join a list): the exact path decides the row
        bool exact = sh.overflow || listed < rank;

        // Fast path (no top-p, or top-p with rank <= 64): every key at or above lo (the largest of the waves'
        // bounds, still at most the K-th largest, and every such key is listed) goes into one 256-bin histogram
        // over [lo, hi], the bins spread over that range so few keys share one. The bin holding the rank-th largest
        // and the bins above it hold few keys; they move to one short list (the bin's own keys also to a second),
        // where wave 0 finds the threshold by counting, applies top-p, and finishes the row.
        constexpr int kTopCap = kSelWaves * 64;   // short-list capacity: indices follow the keys in sortbuf
        uint32_t* bin_keys = &sh.whist[0][0];
        bool fast = !exact && (!a.has_top_p || rank <= 64);
        uint32_t lo = 0u, hi = 0u, bin = 0u, bin_rank = 0u;
        int shift = 0;
        if (fast) {
            for (int w = 0; w < kSelWaves; ++w) {
                lo = max(lo, sh.wlo[w]);
                hi = max(hi, sh.wmax[w]);
            }
            const uint32_t range = hi - lo;
            shift = range < 256u ? 0 : 24 - __clz(range);
#pragma unroll
            for (int s = 0; s < kLaneCap; ++s)
                if (s < lcnt && lk[s] >= lo) atomicAdd(&sh.hist[(lk[s] - lo) >> shift], 1u);
            __syncthreads();
            wave_pick_bin(sh.hist, static_cast<uint32_t>(rank), bin, bin_rank);
            // the same on every wave; a histogram with fewer than rank keys (never expected) goes to the exact path
            const bool picked = bin < 256u;
            const int n_top = picked ? rank - static_cast<int>(bin_rank) + static_cast<int>(sh.hist[bin]) : 0;
            exact = !picked;
            fast = picked && n_top <= kTopCap;
            if (fast) {
                // each lane's entries in the picked bin or above it (and in the bin), one prefix over the wave and
                // one reservation per wave and list, then the lane's entries in order
                int n_take = 0, n_bin = 0;
#pragma unroll
                for (int s = 0; s < kLaneCap; ++s) {
                    const bool in = s < lcnt && lk[s] >= lo;
                    const uint32_t d = (lk[s] - lo) >> shift;
                    n_take += (in && d >= bin) ? 1 : 0;
                    n_bin += (in && d == bin) ? 1 : 0;
                }
                const int incl_t = wave_scan_incl_dpp(n_take);
                const int incl_b = wave_scan_incl_dpp(n_bin);
                int base_t = 0, base_b = 0;
                if (lane == 63) {
                    if (incl_t > 0) base_t = atomicAdd(&sh.count, incl_t);
                    if (incl_b > 0) base_b = atomicAdd(&sh.bin_count, incl_b);
                }
                int pt = __shfl(base_t, 63) + incl_t - n_take;
                int pb = __shfl(base_b, 63) + incl_b - n_bin;
#pragma unroll
                for (int s = 0; s < kLaneCap; ++s) {
                    const uint32_t key = lk[s];
                    const bool in = s < lcnt && key >= lo;
                    const uint32_t d = (key - lo) >> shift;
                    if (in && d >= bin) {
                        sh.sortbuf[pt] = key;
                        sh.sortbuf[kTopCap + pt] = static_cast<uint32_t>(widx[s * 64 + lane]);
                        ++pt;
                        if (d == bin) bin_keys[pb++] = key;
                    }
                }
            }
            __syncthreads();
        }
        if (fast) {
            // Wave 0 finishes the row alone: the threshold, the softmax sum over the kept keys and, for the fused
            // accept, this position's accept test, its race and its record.
            if (wave == 0) {
                const int n_top = sh.count;
                uint32_t kk[kSelWaves];
                int32_t ki[kSelWaves];
#pragma unroll
                for (int w = 0; w < kSelWaves; ++w) {
                    const int c = w * 64 + lane;
                    kk[w] = c < n_top ? sh.sortbuf[c] : 0u;
                    ki[w] = c < n_top ? static_cast<int32_t>(sh.sortbuf[kTopCap + c]) : 0;
                }
                // the fused accept with q as candidate rows: the row's first candidates requested now (hashed
                // after the threshold)
                int32_t qh_id[2] = {-1, -1};
                float qh_pr[2] = {0.f, 0.f};
                if constexpr (MODE == kModeAccept) {
                    const int64_t j = sh.loc[1], L = sh.loc[2];
                    const bool bonus = (j >= L - 1) || (j >= a.k);
                    if (a.q_ids != nullptr && !bonus && a.q_cand <= kQHash / 2)
                        load_q_row_head(a, sh.loc[0] * a.k + j, qh_id, qh_pr);
                }
                // threshold: the largest key of the bin with at least bin_rank keys of the bin at or above it
                const int nb_keys = sh.bin_count;
                uint32_t cand = 0u;
                for (int i = lane; i < nb_keys; i += 64) {
                    const uint32_t ki_key = bin_keys[i];
                    uint32_t ge = 0;
                    for (int jj = 0; jj < nb_keys; ++jj) ge += (bin_keys[jj] >= ki_key) ? 1u : 0u;
                    if (ge >= bin_rank) cand = max(cand, ki_key);
                }
                const uint32_t thr_key = wave_max_u32(cand);
                const float m = nvs::key_float(hi);
                const float mu_f = (m == -INFINITY) ? 0.f : m;
                uint32_t theta_key = thr_key;
                if (a.has_top_p) {
                    // top-p over the rank candidates (rank <= 64): the keys above the threshold (fewer than rank)
                    // sorted into lanes, the threshold repeated up to rank (truncate_logits' -inf beyond it)
                    uint32_t* gbuf = sh.hist;   // free once the short list is formed
                    int g = 0;
#pragma unroll
                    for (int w = 0; w < kSelWaves; ++w) {
                        const bool gt = kk[w] > thr_key;
                        const uint64_t bal = __ballot(gt);
                        if (gt)
                            gbuf[g + static_cast<int>(__builtin_amdgcn_mbcnt_hi(
                                          static_cast<uint32_t>(bal >> 32),
                                          __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(bal), 0u)))] = kk[w];
                        g += __popcll(bal);
                    }
                    compiler_fence_s();
                    const uint32_t sorted = wave_sort_desc(lane < g ? gbuf[lane] : 0u);
                    const uint32_t key_l = lane < g ? sorted : (lane < rank ? thr_key : 0u);
                    const float theta =
                        wave_top_p_threshold64(key_l, rank, K, top_p, nvs::key_float(thr_key));
                    theta_key = (theta == -INFINITY) ? thr_key : nvs::float_key(theta);
                }
                float z = 0.f;
#pragma unroll
                for (int w = 0; w < kSelWaves; ++w)
                    if (kk[w] >= theta_key) z += expf(nvs::key_float(kk[w]) - mu_f);
                z = wave_sum(z);
                if (lane == 0) {
                    sh.fast_m = m;
                    sh.fast_z = z;
                    sh.fast_theta = nvs::key_float(theta_key);
                }
                if constexpr (MODE == kModeAccept) {
                    const int64_t b = sh.loc[0], j = sh.loc[1], L = sh.loc[2];
                    const int kd = a.k;
                    const bool bonus = (j >= L - 1) || (j >= kd);
                    int acc = 0;
                    // candidate rows of q: wave 0 hashes this draft row's tokens into the refinement histograms'
                    // space (free once the threshold is known); rows with more candidates are broadcast instead
                    const bool sparse = a.q_ids != nullptr;
                    const bool whash = sparse && !bonus && a.q_cand <= kQHash / 2;
                    // the kept tokens' noise requested first (index 0 stands in for a pair that is not kept), so
                    // that its round trip overlaps the q lookups below
                    const float* erow = a.noise + b * a.vocab;
                    float qv[kSelWaves], ev[kSelWaves];
                    int32_t tok[kSelWaves];
#pragma unroll
                    for (int w = 0; w < kSelWaves; ++w) {
                        tok[w] = kk[w] >= theta_key ? ki[w] : 0;
                        ev[w] = erow[tok[w]];
                    }
                    if (whash) build_q_hash_wave(a, b * kd + j, sh, qh_id[0], qh_pr[0], qh_id[1], qh_pr[1]);
                    float dq = dec_q;
                    if (sparse && dec_valid) dq = whash ? q_hash_lookup(sh, dec_d) : sparse_q_wave(a, dec_slot, dec_d);
                    if (lane == 0 && dec_valid) {
                        const float sd = scale_logit(dec_x, temp, unit_temp);
                        const float pd = (sel_key(sd) >= theta_key && sel_key(sd) != 0u) ? expf(sd - mu_f) / z : 0.f;
                        acc = (dec_u * dq < pd) ? 1 : 0;
                    }
                    if (bonus) {
#pragma unroll
                        for (int w = 0; w < kSelWaves; ++w) qv[w] = 0.f;
                    } else if (whash) {
#pragma unroll
                        for (int w = 0; w < kSelWaves; ++w) qv[w] = q_hash_lookup(sh, tok[w]);
                    } else if (sparse) {
                        sparse_q_wave8(a, b * kd + j, tok, qv);
                    } else {
                        const float* qrow = a.q + (b * kd + j) * a.vocab;
#pragma unroll
                        for (int w = 0; w < kSelWaves; ++w) qv[w] = qrow[tok[w]];
                    }
                    uint64_t best = 0;
#pragma unroll
                    for (int w = 0; w < kSelWaves; ++w) {
                        if (kk[w] < theta_key) continue;
                        const float p = expf(nvs::key_float(kk[w]) - mu_f) / z;
                        const float wgt = bonus ? p : fmaxf(p - qv[w], 0.f);
                        const float score = wgt / ev[w];
                        const uint64_t k64 = (static_cast<uint64_t>(nvs::float_key(score)) << 32) |
                                             static_cast<uint64_t>(0xffffffffu - static_cast<uint32_t>(ki[w]));
                        best = best > k64 ? best : k64;
                    }
                    best = wave_max_u64(best);
                    if (lane == 0) {
                        PosRecord r;
                        r.m = m;
                        r.z = z;
                        r.theta = nvs::key_float(theta_key);
                        r.temp = temp;
                        r.flags = 0;
                        r.acc = acc;
                        int64_t winner = 0;
                        if (best != 0) {
                            const float score = nvs::key_float(static_cast<uint32_t>(best >> 32));
                            // all weights zero: torch's argmax over the zero vector is index 0
                            winner = (score > 0.f) ? static_cast<int64_t>(0xffffffffu - static_cast<uint32_t>(best))
                                                   : int64_t{0};
                        }
                        r.race = winner;
                        store_record(a.rec + t, r);
                        if (sh.found) {
                            // every position of the row that exists counts once (see row_positions)
                            sh.last = count_position(&a.counters[b], row_positions(a, sh.loc[3], L)) ? 1 : 0;
                        }
                    }
                }
            }
            __syncthreads();
            rs.m = sh.fast_m;
            rs.z = sh.fast_z;
            rs.theta = sh.fast_theta;
            rs.dense = false;
            record_done = true;
            kept_source = kKeptInShortList;
        } else {
        if (!exact) {
            // the lanes' lists, one after another (wave by wave, lane by lane), at the front of the buffer
            int off = 0, total = 0;
            for (int w = 0; w < kSelWaves; ++w) {
                off += (w < wave) ? sh.wcount[w] : 0;
                total += sh.wcount[w];
            }
            off += wave_scan_incl_dpp(lcnt) - lcnt;
            uint32_t kk[kLaneCap];
            int32_t ii[kLaneCap];
#pragma unroll
            for (int s = 0; s < kLaneCap; ++s) {
                kk[s] = s < lcnt ? wkey[s * 64 + lane] : 0u;
                ii[s] = s < lcnt ? widx[s * 64 + lane] : 0;
            }
            __syncthreads();
#pragma unroll
            for (int s = 0; s < kLaneCap; ++s) {
                if (s < lcnt) {
                    sh.ckey[off + s] = kk[s];
                    sh.cidx[off + s] = ii[s];
                }
            }
            if (threadIdx.x == 0) sh.count = total;
        }
        __syncthreads();
        if (exact) {
            rs = exact_row_stats<DT, VEC, WIDE>(a, row, temp, unit_temp, rank, K, top_p, sh);
        } else {
            kept_source = kKeptInLists;
            const int n = sh.count;
            auto each = [&](auto&& fn) {
                for (int c = threadIdx.x; c < n; c += blockDim.x) fn(sh.ckey[c]);
            };
            uint32_t ng, ne;
            const uint32_t thr_key = radix_select(each, static_cast<uint32_t>(rank), sh, &ng, &ne);
            uint32_t mk = 0u;
            for (int c = threadIdx.x; c < n; c += blockDim.x) mk = max(mk, sh.ckey[c]);
            mk = block_max_u32(mk, sh);
            rs.m = nvs::key_float(mk);
            const float thr = nvs::key_float(thr_key);
            rs.theta = thr;
            if (a.has_top_p) {
                __shared__ int gcount;
                if (threadIdx.x == 0) gcount = 0;
                __syncthreads();
                for (int c = threadIdx.x; c < n; c += blockDim.x)
                    if (sh.ckey[c] > thr_key) sh.sortbuf[atomicAdd(&gcount, 1)] = sh.ckey[c];
                __syncthreads();
                const int g = gcount;
                block_sort_desc(sh, g);
                for (int i = g + threadIdx.x; i < rank; i += blockDim.x) sh.sortbuf[i] = thr_key;
                __syncthreads();
                rs.theta = top_p_threshold(sh, rank, K, top_p, thr);
            }
            const uint32_t theta_key = nvs::float_key(rs.theta);
            float z = 0.f;
            for (int c = threadIdx.x; c < n; c += blockDim.x)
                if (sh.ckey[c] >= theta_key) z += expf(nvs::key_float(sh.ckey[c]) - rs.m);
            rs.z = block_sum(z, sh);
            rs.dense = false;
        }
        }
    }

    const uint32_t theta_key = rs.theta == -INFINITY ? 0u : nvs::float_key(rs.theta);
    const float mu = (rs.m == -INFINITY) ? 0.f : rs.m;

    if constexpr (MODE == kModeMarkov) {
        markov_tail<DT, VEC>(a, t, row, temp, unit_temp, theta_key, kept_source, sh);
        return;
    } else if constexpr (MODE == kModeProbs || MODE == kModeTruncate) {
        float* orow = a.out + t * a.out_stride;
        if (!rs.dense && kept_source != kKeptInRow && theta_key != 0u) {
            // Every kept value (key >= theta_key > 0: NaN is never kept) is in LDS, in the short list or the lane
            // lists. The row is filled with the value of an element outside the kept set (probability 0, logit
            // -inf) with 16-byte stores, then the kept values are written over it: the logits are not read again.
            const float fill = MODE == kModeProbs ? 0.f : -INFINITY;
            const int64_t n4 = (reinterpret_cast<uintptr_t>(orow) & 15u) == 0 ? a.vocab / 4 : 0;
            const float4 f4 = make_float4(fill, fill, fill, fill);
            for (int64_t i = threadIdx.x; i < n4; i += kSelThreads) reinterpret_cast<float4*>(orow)[i] = f4;
            for (int64_t e = n4 * 4 + threadIdx.x; e < a.vocab; e += kSelThreads) orow[e] = fill;
            __syncthreads();   // the fill stores are performed before any kept value is written over them
            const bool short_list = kept_source == kKeptInShortList;
            const int n = short_list ? sh.count : min(sh.count, kCap);
            for (int c = threadIdx.x; c < n; c += kSelThreads) {
                const uint32_t key = short_list ? sh.sortbuf[c] : sh.ckey[c];
                if (key < theta_key) continue;
                const int64_t e = short_list ? static_cast<int64_t>(sh.sortbuf[kSelWaves * 64 + c])
                                             : static_cast<int64_t>(sh.cidx[c]);
                const float s = nvs::key_float(key);
                if constexpr (MODE == kModeProbs) {
                    orow[e] = expf(s - mu) / rs.z;
                } else {
                    orow[e] = s;
                }
            }
            return;
        }
        for (int64_t e0 = 0; e0 < a.vocab; e0 += kBatch) {
            float v[kVpt];
            load_vals<DT, VEC>(row, e0, a.vocab, v);
#pragma unroll
            for (int vi = 0; vi < kVpt; ++vi) {
                const int64_t e = val_index<DT>(e0, vi);
                if (e >= a.vocab) continue;
                const float s = scale_logit(v[vi], temp, unit_temp);
                const bool kept = sel_key(s) >= theta_key;
                if constexpr (MODE == kModeProbs) {
                    orow[e] = kept ? expf(s - mu) / rs.z : 0.f;
                } else {
                    orow[e] = kept ? s : -INFINITY;
                }
            }
        }
        return;
    } else {
        // ---- fused accept: this position's accept test and race
        const int64_t b = sh.loc[0], j = sh.loc[1], L = sh.loc[2];
        if (record_done) {
            if (!sh.last) return;
            finish_row<DT>(a, b, sh.loc[3], L, sh);
            return;
        }
        const int kd = a.k;
        const bool bonus = (j >= L - 1) || (j >= kd);
        int acc = 0;
        // candidate rows of q: a hash of this draft row's tokens in LDS (the race below and the accept test look
        // up q there), or a scan of the row when it has too many candidates for the hash
        const bool sparse = a.q_ids != nullptr;
        const bool hashed = sparse && !bonus && a.q_cand <= kQHash / 2;
        if (hashed) build_q_hash(a, b * kd + j, sh);
        auto q_at = [&](int64_t i) -> float {
            if (!sparse) return a.q[(b * kd + j) * a.vocab + i];
            return hashed ? q_hash_lookup(sh, i) : sparse_q_scan(a, b * kd + j, i);
        };
        if (threadIdx.x == 0 && dec_valid) {
            const float sd = scale_logit(dec_x, temp, unit_temp);
            const float pd = (sel_key(sd) >= theta_key && sel_key(sd) != 0u) ? expf(sd - mu) / rs.z : 0.f;
            const float dq = sparse ? q_at(dec_d) : dec_q;
            acc = (dec_u * dq < pd) ? 1 : 0;
        }
        uint64_t best = 0;
        if (!rs.dense) {
            const int n = min(sh.count, kCap);
            const float* erow = a.noise + b * a.vocab;
            for (int c = threadIdx.x; c < n; c += blockDim.x) {
                const uint32_t key = sh.ckey[c];
                if (key < theta_key) continue;
                const int64_t i = sh.cidx[c];
                const float p = expf(nvs::key_float(key) - mu) / rs.z;
                const float w = bonus ? p : fmaxf(p - q_at(i), 0.f);
                const float score = w / erow[i];
                const uint64_t k64 = (static_cast<uint64_t>(nvs::float_key(score)) << 32) |
                                     static_cast<uint64_t>(0xffffffffu - static_cast<uint32_t>(i));
                best = best > k64 ? best : k64;
            }
        }
        best = block_max_u64(best, sh);
        if (threadIdx.x == 0) {
            PosRecord r;
            r.m = rs.m;
            r.z = rs.z;
            r.theta = rs.theta;
            r.temp = temp;
            r.flags = rs.dense ? kFlagDense : 0;
            r.acc = acc;
            int64_t winner = 0;
            if (!rs.dense && best != 0) {
                const float score = nvs::key_float(static_cast<uint32_t>(best >> 32));
                // all weights zero: torch's argmax over the zero vector is index 0
                winner = (score > 0.f) ? static_cast<int64_t>(0xffffffffu - static_cast<uint32_t>(best))
                                       : int64_t{0};
            }
            r.race = winner;
            store_record(a.rec + t, r);
            // count the position; the row's last position to arrive finishes the row
            if (sh.found) sh.last = count_position(&a.counters[b], row_positions(a, sh.loc[3], L)) ? 1 : 0;
        }
        __syncthreads();
        if (!sh.last) return;
        finish_row<DT>(a, b, sh.loc[3], L, sh);
    }
}

__device__ __forceinline__ int64_t row_start(const int64_t* lens, int64_t b, int k) {
    // exclusive prefix of lens over rows < b (workgroup reduction)
    __shared__ int64_t part[4];
    if (lens == nullptr) return b * (k + 1);
    int64_t s = 0;
    for (int64_t i = threadIdx.x; i < b; i += blockDim.x) s += lens[i];
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = s;
    __syncthreads();
    int64_t tot = 0;
    for (int w = 0; w < (int)(blockDim.x >> 6); ++w) tot += part[w];
    return tot;
}

// ---------------------------------------------------------------- dense race kernels

struct RaceArgs {
    // w(i) = bonus ? p[prow, i] : max(p[prow, i] - q[qrow, i], 0)   (accept)   or   w[r, i]   (race)
    const float* p;
    int64_t p_stride;
    const float* q;
    const float* noise;
    int64_t noise_stride;
    const int64_t* drafts;
    const int64_t* lens;
    const float* uniforms;
    int64_t rows;
    int64_t n_pos;
    int k;
    int64_t vocab;
    int n_chunks;
    uint64_t* partial;  // [rows, n_chunks]
    int* counters;      // [rows] chunks of the row finished; zero between calls
    int64_t* n_accept;
    int64_t* out;
};

// Accepted prefix of row b over dense p (accept_random_varlen's gathers, spec_sampler.py:134-143).
__device__ int64_t accepted_prefix(const RaceArgs& a, int64_t b, int64_t start, int64_t L) {
    // Draft n is tested only when every draft before it was accepted (spec_sampler.py:136-141): the prefix is the
    // number of leading accepted drafts among the first lim = min(L - 1, k, n_pos - start). Wave 0 tests them all
    // at once, one lane per draft (two dependent loads: the draft, then p and q at it), and counts the leading
    // accepted lanes; rows with more than 64 drafts are walked in steps of 64.
    __shared__ int64_t n_sh;
    if (threadIdx.x < 64) {
        const int64_t lim = min(min(L - 1, static_cast<int64_t>(a.k)), a.n_pos - start);
        int64_t n = 0;
        for (int64_t j0 = 0; j0 < lim; j0 += 64) {
            const int64_t j = j0 + threadIdx.x;
            bool acc = false;
            if (j < lim) {
                const int64_t d = a.drafts[b * a.k + j];
                const float u = a.uniforms[b * a.k + j];
                if (d >= 0 && d < a.vocab) {   // an out-of-vocabulary draft is never accepted
                    const float pd = a.p[(start + j) * a.p_stride + d];
                    const float qd = a.q[(b * a.k + j) * a.vocab + d];
                    acc = u * qd < pd;
                }
            }
            const uint64_t rejected = ~__ballot(acc);
            if (rejected != 0ull) {
                n = j0 + __builtin_ctzll(rejected);
                break;
            }
            n = j0 + 64;
        }
        if (threadIdx.x == 0) n_sh = min(n, max(lim, int64_t{0}));
    }
    __syncthreads();
    return n_sh;
}

// One workgroup = (row r, chunk c of kRaceChunk elements): the best (score, -index) key of the chunk. VEC (every
// row 16-byte aligned, vocab a multiple of 4): each thread takes kRacePer 16-byte pieces of each array, all loads
// issued before any is used, the noise first (it does not depend on the accepted prefix), from addresses clamped
// into the chunk; pieces past the chunk are loaded but not scored.
template <bool kAccept, bool VEC>
__global__ __launch_bounds__(256) void race_chunk_kernel(RaceArgs a) {
    __shared__ uint64_t red[4];
    const int64_t r = blockIdx.x;   // rows on x (up to 2^31), vocabulary chunks on y
    const int c = blockIdx.y;
    const float* erow = a.noise + r * a.noise_stride;
    const int64_t i0 = static_cast<int64_t>(c) * kRaceChunk;
    const int64_t i1 = min(i0 + kRaceChunk, a.vocab);
    float4 ev[kRacePer];
    if constexpr (VEC) {
#pragma unroll
        for (int m = 0; m < kRacePer; ++m) {
            const int64_t j = min((i0 >> 2) + threadIdx.x + 256 * m, (i1 >> 2) - 1);
            ev[m] = reinterpret_cast<const float4*>(erow)[j];
        }
    }
    const float* wrow;
    const float* qrow = nullptr;
    bool bonus = true;
    if constexpr (kAccept) {
        const int64_t start = row_start(a.lens, r, a.k);
        const int64_t L = a.lens != nullptr ? a.lens[r] : a.k + 1;
        const int64_t n = accepted_prefix(a, r, start, L);
        bonus = (n == L - 1);
        wrow = a.p + min(start + n, a.n_pos - 1) * a.p_stride;
        qrow = a.q + (r * a.k + (n < a.k - 1 ? n : a.k - 1)) * a.vocab;
        if (c == 0 && threadIdx.x == 0) a.n_accept[r] = n;
    } else {
        wrow = a.p + r * a.p_stride;
    }
    auto key_of = [](float w, float e, int64_t i) {
        const float score = w / e;
        return (static_cast<uint64_t>(nvs::float_key(score)) << 32) |
               static_cast<uint64_t>(0xffffffffu - static_cast<uint32_t>(i));
    };
    uint64_t best = 0;
    if constexpr (VEC) {
        float4 wv[kRacePer], qv[kRacePer];
#pragma unroll
        for (int m = 0; m < kRacePer; ++m) {
            const int64_t j = min((i0 >> 2) + threadIdx.x + 256 * m, (i1 >> 2) - 1);
            wv[m] = reinterpret_cast<const float4*>(wrow)[j];
            // a bonus row has no q; its pieces are then the w row's again (never used)
            if constexpr (kAccept) qv[m] = reinterpret_cast<const float4*>(!bonus ? qrow : wrow)[j];
        }
#pragma unroll
        for (int m = 0; m < kRacePer; ++m) {
            const int64_t j = (i0 >> 2) + threadIdx.x + 256 * m;
            if (j >= (i1 >> 2)) continue;
            const float w4[4] = {wv[m].x, wv[m].y, wv[m].z, wv[m].w};
            const float q4[4] = {kAccept ? qv[m].x : 0.f, kAccept ? qv[m].y : 0.f, kAccept ? qv[m].z : 0.f,
                                 kAccept ? qv[m].w : 0.f};
            const float e4[4] = {ev[m].x, ev[m].y, ev[m].z, ev[m].w};
#pragma unroll
            for (int l = 0; l < 4; ++l) {
                const float w = (kAccept && !bonus) ? fmaxf(w4[l] - q4[l], 0.f) : w4[l];
                const uint64_t k64 = key_of(w, e4[l], 4 * j + l);
                best = best > k64 ? best : k64;
            }
        }
    } else {
        for (int64_t i = i0 + threadIdx.x; i < i1; i += blockDim.x) {
            float w = wrow[i];
            if (kAccept && !bonus) w = fmaxf(w - qrow[i], 0.f);
            const uint64_t k64 = key_of(w, erow[i], i);
            best = best > k64 ? best : k64;
        }
    }
    best = wave_max_u64(best);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = best;
    __syncthreads();
    if (threadIdx.x < 64) {
        // the row's last chunk to finish picks the winner over the row's chunk keys (the accepted prefix was
        // written by the row's chunk 0)
        uint64_t all = 0;
        for (int w = 0; w < 4; ++w) all = red[w] > all ? red[w] : all;
        uint64_t win = 0;
        if (finish_race_chunk(a.partial + r * a.n_chunks, a.n_chunks, c, all, a.counters + r, win) &&
            threadIdx.x == 0)
            a.out[r] = static_cast<int64_t>(0xffffffffu - static_cast<uint32_t>(win));
    }
}

// ---------------------------------------------------------------- greedy

template <int DT, bool VEC>
__global__ __launch_bounds__(kSelThreads) void argmax_kernel(const void* logits, int64_t row_stride, int64_t vocab,
                                                             int64_t* tokens) {
    __shared__ uint64_t red[kSelWaves];
    const int64_t t = blockIdx.x;
    const char* row = static_cast<const char*>(logits) + t * row_stride * nvs::dtype_size(DT);
    uint64_t best = 0;
    for (int64_t e0 = 0; e0 < vocab; e0 += kBatch) {
        float v[kVpt];
        load_vals<DT, VEC>(row, e0, vocab, v);
#pragma unroll
        for (int vi = 0; vi < kVpt; ++vi) {
            const int64_t e = val_index<DT>(e0, vi);
            if (e >= vocab) continue;
            // torch's argmax: NaN counts as the maximum; first index on ties
            const uint32_t key = (v[vi] != v[vi]) ? 0xffffffffu : nvs::float_key(v[vi]);
            const uint64_t k64 = (static_cast<uint64_t>(key) << 32) |
                                 static_cast<uint64_t>(0xffffffffu - static_cast<uint32_t>(e));
            best = best > k64 ? best : k64;
        }
    }
    best = wave_max_u64(best);
    if (lane_id() == 0) red[threadIdx.x >> 6] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint64_t all = 0;
        for (int w = 0; w < kSelWaves; ++w) all = red[w] > all ? red[w] : all;
        tokens[t] = static_cast<int64_t>(0xffffffffu - static_cast<uint32_t>(all));
    }
}

// One workgroup per batch row: the row's first position (a reduction over the lengths before it), then the
// accepted prefix and the token after it.
__global__ __launch_bounds__(256) void greedy_finalize_kernel(const int64_t* tokens, const int64_t* drafts,
                                                              const int64_t* lens, int64_t batch, int64_t n_pos,
                                                              int k, int64_t* n_accept, int64_t* tail) {
    const int64_t b = blockIdx.x;
    const int64_t start = row_start(lens, b, k);
    if (threadIdx.x != 0) return;
    const int64_t L = lens != nullptr ? lens[b] : k + 1;
    int64_t n = 0;
    while (n < L - 1 && n < k && start + n < n_pos && tokens[start + n] == drafts[b * k + n]) ++n;
    n_accept[b] = n;
    tail[b] = tokens[min(start + n, n_pos - 1)];
}

// ---------------------------------------------------------------- host side

int check_dtype(int dt) {
    NVS_CHECK(dt == NVS_DTYPE_F32 || dt == NVS_DTYPE_BF16 || dt == NVS_DTYPE_F16, NVS_ERR_INVALID,
              "sampler: unknown logits dtype %d", dt);
    return NVS_OK;
}

// Any window width is served: windows above kMaxTopK take the exact path over the row (wide_row_stats).
int check_topk(int max_top_k) {
    NVS_CHECK(max_top_k >= 0, NVS_ERR_INVALID, "sampler: max_top_k %d is negative", max_top_k);
    return NVS_OK;
}

// Rows qualify for the 16-byte streaming loads when every row starts 16-byte aligned and the vocabulary is a
// whole number of 16-byte pieces.
bool vector_rows(const void* base, int64_t row_stride, int64_t vocab, int dt) {
    const int es = nvs::dtype_size(dt);
    const int w = 16 / es;
    return nvs::aligned16(base) && (row_stride * es) % 16 == 0 && vocab % w == 0;
}

template <int DT, int MODE>
void launch_select_dt(const SelArgs& a, bool vec, hipStream_t s) {
    const dim3 grid(static_cast<unsigned>(a.n_pos));
    // windows wider than the candidate lists take the wide instantiation (the Markov draw never has them)
    if constexpr (MODE != kModeMarkov) {
        if (a.max_top_k > kMaxTopK && a.vocab > kMaxTopK) {
            if (vec) {
                hipLaunchKernelGGL((select_kernel<DT, MODE, true, true>), grid, dim3(kSelThreads), 0, s, a);
            } else {
                hipLaunchKernelGGL((select_kernel<DT, MODE, false, true>), grid, dim3(kSelThreads), 0, s, a);
            }
            return;
        }
    }
    if (vec) {
        hipLaunchKernelGGL((select_kernel<DT, MODE, true, false>), grid, dim3(kSelThreads), 0, s, a);
    } else {
        hipLaunchKernelGGL((select_kernel<DT, MODE, false, false>), grid, dim3(kSelThreads), 0, s, a);
    }
}

template <int MODE>
int launch_select(int dt, const SelArgs& a, hipStream_t s) {
    const bool vec = vector_rows(a.logits, a.row_stride, a.vocab, dt);
    switch (dt) {
        case NVS_DTYPE_F32: launch_select_dt<NVS_DTYPE_F32, MODE>(a, vec, s); break;
        case NVS_DTYPE_BF16: launch_select_dt<NVS_DTYPE_BF16, MODE>(a, vec, s); break;
        default: launch_select_dt<NVS_DTYPE_F16, MODE>(a, vec, s); break;
    }
    return nvs::check_launch("sampler select kernel");
}

template <int DT>
void launch_argmax(const void* logits, int64_t row_stride, int64_t n_pos, int64_t vocab, int64_t* tokens,
                   hipStream_t s) {
    const dim3 grid(static_cast<unsigned>(n_pos));
    if (vector_rows(logits, row_stride, vocab, DT)) {
        hipLaunchKernelGGL((argmax_kernel<DT, true>), grid, dim3(kSelThreads), 0, s, logits, row_stride, vocab, tokens);
    } else {
        hipLaunchKernelGGL((argmax_kernel<DT, false>), grid, dim3(kSelThreads), 0, s, logits, row_stride, vocab,
                           tokens);
    }
}

int64_t race_chunks(int64_t vocab) { return (vocab + kRaceChunk - 1) / kRaceChunk; }

}  // namespace

// ================================================================ entry points

extern "C" int nvs_probs_from_logits_workspace_size(int64_t n_pos, int64_t vocab, int max_top_k, size_t* bytes) {
    nvs::clear_error();
    NVS_CHECK(bytes != nullptr, NVS_ERR_INVALID, "probs_from_logits_workspace_size: bytes is NULL");
    NVS_CHECK(n_pos >= 0 && vocab >= 0, NVS_ERR_INVALID, "probs_from_logits: negative size");
    const int st = check_topk(max_top_k);
    if (st != NVS_OK) return st;
    *bytes = 0;
    return NVS_OK;
}

static int common_select_checks(const void* logits, int64_t row_stride, int64_t n_pos, int64_t vocab,
                                int64_t pos_per_param, int max_top_k, const int64_t* top_k) {
    NVS_CHECK(n_pos >= 0 && vocab > 0, NVS_ERR_INVALID, "sampler: bad sizes n_pos=%lld vocab=%lld",
              (long long)n_pos, (long long)vocab);
    NVS_CHECK(vocab < 0x7fffffffLL, NVS_ERR_UNSUPPORTED, "sampler: vocab %lld too large", (long long)vocab);
    NVS_CHECK(row_stride >= vocab, NVS_ERR_INVALID, "sampler: row stride %lld < vocab %lld", (long long)row_stride,
              (long long)vocab);
    NVS_CHECK(pos_per_param >= 1, NVS_ERR_INVALID, "sampler: pos_per_param must be >= 1");
    NVS_CHECK(n_pos <= 0x7fffffffLL, NVS_ERR_UNSUPPORTED, "sampler: too many positions");
    NVS_CHECK(n_pos == 0 || logits != nullptr, NVS_ERR_INVALID, "sampler: logits is NULL");
    NVS_CHECK(max_top_k == 0 || top_k != nullptr, NVS_ERR_INVALID, "sampler: max_top_k > 0 needs top_k");
    return check_topk(max_top_k);
}

extern "C" int nvs_probs_from_logits(const void* logits, int logits_dtype, int64_t logits_row_stride, int64_t n_pos,
                                     int64_t vocab, int64_t pos_per_param, const float* temperatures,
                                     const int64_t* top_k, const float* top_p, int max_top_k, int has_top_p,
                                     float* probs, void* workspace, size_t workspace_bytes, void* stream) {
    (void)workspace;
    (void)workspace_bytes;
    nvs::clear_error();
    int st = check_dtype(logits_dtype);
    if (st != NVS_OK) return st;
    st = common_select_checks(logits, logits_row_stride, n_pos, vocab, pos_per_param, max_top_k, top_k);
    if (st != NVS_OK) return st;
    NVS_CHECK(temperatures != nullptr, NVS_ERR_INVALID, "probs_from_logits: temperatures is NULL (greedy batch)");
    NVS_CHECK(!has_top_p || top_p != nullptr, NVS_ERR_INVALID, "probs_from_logits: has_top_p needs top_p");
    NVS_CHECK(n_pos == 0 || probs != nullptr, NVS_ERR_INVALID, "probs_from_logits: probs is NULL");
    if (n_pos == 0) return NVS_OK;
    SelArgs a{};
    a.logits = logits;
    a.row_stride = logits_row_stride;
    a.n_pos = n_pos;
    a.vocab = vocab;
    a.temps = temperatures;
    a.top_k = max_top_k > 0 ? top_k : nullptr;
    a.top_p = top_p;
    a.max_top_k = max_top_k;
    a.has_top_p = has_top_p && max_top_k > 0;
    a.pos_per_param = pos_per_param;
    a.out = probs;
    a.out_stride = vocab;
    return launch_select<kModeProbs>(logits_dtype, a, static_cast<hipStream_t>(stream));
}

extern "C" int nvs_truncate_logits(const float* scaled, int64_t scaled_row_stride, int64_t n_pos, int64_t vocab,
                                   int64_t pos_per_param, const int64_t* top_k, const float* top_p, int max_top_k,
                                   int has_top_p, float* out, void* workspace, size_t workspace_bytes,
                                   void* stream) {
    (void)workspace;
    (void)workspace_bytes;
    nvs::clear_error();
    int st = common_select_checks(scaled, scaled_row_stride, n_pos, vocab, pos_per_param, max_top_k, top_k);
    if (st != NVS_OK) return st;
    NVS_CHECK(!has_top_p || top_p != nullptr, NVS_ERR_INVALID, "truncate_logits: has_top_p needs top_p");
    NVS_CHECK(n_pos == 0 || out != nullptr, NVS_ERR_INVALID, "truncate_logits: out is NULL");
    if (n_pos == 0) return NVS_OK;
    SelArgs a{};
    a.logits = scaled;
    a.row_stride = scaled_row_stride;
    a.n_pos = n_pos;
    a.vocab = vocab;
    a.temps = nullptr;
    a.top_k = max_top_k > 0 ? top_k : nullptr;
    a.top_p = top_p;
    a.max_top_k = max_top_k;
    a.has_top_p = has_top_p && max_top_k > 0;
    a.pos_per_param = pos_per_param;
    a.out = out;
    a.out_stride = vocab;
    return launch_select<kModeTruncate>(NVS_DTYPE_F32, a, static_cast<hipStream_t>(stream));
}

// Segments of the split Markov draw for a row of `vocab` values: (segments, values per segment, a multiple of 8).
static void markov_segments(int64_t vocab, int* n_seg, int* seg_len) {
    int64_t segs = (vocab + kSegKeys - 1) / kSegKeys;
    int64_t len = (vocab + segs - 1) / segs;
    len = (len + 7) / 8 * 8;
    segs = (vocab + len - 1) / len;
    *n_seg = static_cast<int>(segs);
    *seg_len = static_cast<int>(len);
}

static bool markov_split(int64_t vocab, int num_candidates) {
    int n_seg, seg_len;
    markov_segments(vocab, &n_seg, &seg_len);
    // the merge keeps the row's lists in half the pair space and the segments' counts in the lanes of a wave
    return num_candidates <= kSplitMaxCand && n_seg <= 64 &&
           static_cast<int64_t>(n_seg) * num_candidates <= kPairCap / 2;
}

template <int DT>
static void launch_markov_split(const MarkovSplitArgs& a, bool vec, hipStream_t s) {
    const dim3 grid(static_cast<unsigned>(a.n_seg), static_cast<unsigned>(a.batch));
    if (vec && a.bias) {
        hipLaunchKernelGGL((markov_draw_kernel<DT, true, true>), grid, dim3(kSelThreads), 0, s, a);
    } else if (vec) {
        hipLaunchKernelGGL((markov_draw_kernel<DT, true, false>), grid, dim3(kSelThreads), 0, s, a);
    } else if (a.bias) {
        hipLaunchKernelGGL((markov_draw_kernel<DT, false, true>), grid, dim3(kSelThreads), 0, s, a);
    } else {
        hipLaunchKernelGGL((markov_draw_kernel<DT, false, false>), grid, dim3(kSelThreads), 0, s, a);
    }
}

extern "C" int nvs_markov_draw_workspace_size(int64_t batch, int64_t vocab, int num_candidates, size_t* bytes) {
    nvs::clear_error();
    NVS_CHECK(bytes != nullptr && batch >= 0 && vocab > 0 && num_candidates >= 1, NVS_ERR_INVALID,
              "markov_draw_workspace_size: bad arguments");
    int n_seg, seg_len;
    markov_segments(vocab, &n_seg, &seg_len);
    // the segments' pairs [batch, n_seg, n_cand] u64, then their counts [batch, n_seg] int32
    *bytes = markov_split(vocab, num_candidates)
                 ? static_cast<size_t>(batch) * n_seg * (num_candidates * sizeof(uint64_t) + sizeof(int32_t)) : 0;
    return NVS_OK;
}

extern "C" int nvs_markov_draw(const void* logits, int logits_dtype, int64_t logits_row_stride, const void* bias,
                               int64_t bias_row_stride, int64_t batch, int64_t vocab, const float* temperatures,
                               const int64_t* top_k, const float* top_p, int max_top_k, int has_top_p,
                               int num_candidates, const float* noise, int64_t noise_row_stride, int32_t* cand_ids,
                               float* cand_probs, int64_t cand_row_stride, int64_t* draws, int64_t draws_stride,
                               int32_t* row_counters, void* workspace, size_t workspace_bytes, void* stream) {
    nvs::clear_error();
    int st = check_dtype(logits_dtype);
    if (st != NVS_OK) return st;
    st = common_select_checks(logits, logits_row_stride, batch, vocab, 1, max_top_k, top_k);
    if (st != NVS_OK) return st;
    NVS_CHECK(max_top_k >= 1, NVS_ERR_INVALID, "markov_draw: candidate rows need top-k (max_top_k >= 1)");
    NVS_CHECK(max_top_k <= kMaxTopK, NVS_ERR_UNSUPPORTED, "markov_draw: max_top_k %d above %d", max_top_k, kMaxTopK);
    NVS_CHECK(num_candidates <= kMaxCandidates, NVS_ERR_UNSUPPORTED,
              "markov_draw: num_candidates %d above %d", num_candidates, kMaxCandidates);
    NVS_CHECK(num_candidates >= 1 && num_candidates >= min(static_cast<int64_t>(max_top_k), vocab), NVS_ERR_INVALID,
              "markov_draw: num_candidates %d below min(max_top_k, vocab): the candidates must hold the top-k",
              num_candidates);
    NVS_CHECK(temperatures != nullptr, NVS_ERR_INVALID, "markov_draw: temperatures is NULL (greedy rows use argmax)");
    NVS_CHECK(!has_top_p || top_p != nullptr, NVS_ERR_INVALID, "markov_draw: has_top_p needs top_p");
    NVS_CHECK(batch == 0 || (noise && cand_ids && cand_probs && draws), NVS_ERR_INVALID,
              "markov_draw: null noise, cand_ids, cand_probs or draws");
    NVS_CHECK(noise_row_stride >= num_candidates && cand_row_stride >= num_candidates, NVS_ERR_INVALID,
              "markov_draw: a row stride is shorter than num_candidates");
    NVS_CHECK(draws_stride >= 1, NVS_ERR_INVALID, "markov_draw: draws_stride must be >= 1");
    NVS_CHECK(bias == nullptr || bias_row_stride >= vocab, NVS_ERR_INVALID, "markov_draw: bias row stride < vocab");
    NVS_CHECK(batch <= 65535, NVS_ERR_UNSUPPORTED, "markov_draw: batch %lld above 65535", (long long)batch);
    if (batch == 0) return NVS_OK;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (markov_split(vocab, num_candidates)) {
        MarkovSplitArgs m{};
        markov_segments(vocab, &m.n_seg, &m.seg_len);
        const size_t pair_bytes = static_cast<size_t>(batch) * m.n_seg * num_candidates * sizeof(uint64_t);
        const size_t need = pair_bytes + static_cast<size_t>(batch) * m.n_seg * sizeof(int32_t);
        NVS_CHECK(workspace != nullptr && workspace_bytes >= need, NVS_ERR_WORKSPACE,
                  "markov_draw: workspace of %zu bytes needed, %zu given", need, workspace_bytes);
        NVS_CHECK(row_counters != nullptr, NVS_ERR_INVALID,
                  "markov_draw: the split draw needs row_counters (int32 [batch], zero between calls)");
        m.counters = row_counters;
        m.logits = logits;
        m.row_stride = logits_row_stride;
        m.bias = bias;
        m.bias_stride = bias_row_stride;
        m.batch = batch;
        m.vocab = vocab;
        m.temps = temperatures;
        m.top_k = top_k;
        m.top_p = top_p;
        m.max_top_k = max_top_k;
        m.has_top_p = has_top_p;
        m.n_cand = num_candidates;
        m.pairs = static_cast<uint64_t*>(workspace);
        m.seg_counts = reinterpret_cast<int*>(static_cast<unsigned char*>(workspace) + pair_bytes);
        m.noise = noise;
        m.noise_stride = noise_row_stride;
        m.cand_ids = cand_ids;
        m.cand_probs = cand_probs;
        m.cand_stride = cand_row_stride;
        m.draws = draws;
        m.draws_stride = draws_stride;
        const bool vec = vector_rows(logits, logits_row_stride, vocab, logits_dtype) &&
                         (bias == nullptr || vector_rows(bias, bias_row_stride, vocab, logits_dtype));
        switch (logits_dtype) {
            case NVS_DTYPE_F32: launch_markov_split<NVS_DTYPE_F32>(m, vec, s); break;
            case NVS_DTYPE_BF16: launch_markov_split<NVS_DTYPE_BF16>(m, vec, s); break;
            default: launch_markov_split<NVS_DTYPE_F16>(m, vec, s); break;
        }
        return nvs::check_launch("markov draw kernel");
    }
    // more candidates than the split draw takes: one workgroup per sequence, on logits the caller has biased
    NVS_CHECK(bias == nullptr, NVS_ERR_UNSUPPORTED,
              "markov_draw: %d candidates take the unsplit draw, which needs the bias added beforehand",
              num_candidates);
    SelArgs a{};
    a.logits = logits;
    a.row_stride = logits_row_stride;
    a.n_pos = batch;
    a.vocab = vocab;
    a.temps = temperatures;
    a.top_k = top_k;
    a.top_p = top_p;
    a.max_top_k = max_top_k;
    a.has_top_p = has_top_p;
    a.pos_per_param = 1;
    a.noise = noise;
    a.noise_stride = noise_row_stride;
    a.n_cand = num_candidates;
    a.cand_ids = cand_ids;
    a.cand_probs = cand_probs;
    a.cand_stride = cand_row_stride;
    a.draws = draws;
    a.draws_stride = draws_stride;
    return launch_select<kModeMarkov>(logits_dtype, a, s);
}

extern "C" int nvs_race_workspace_size(int64_t n_rows, int64_t vocab, size_t* bytes) {
    nvs::clear_error();
    NVS_CHECK(bytes != nullptr && n_rows >= 0 && vocab >= 0, NVS_ERR_INVALID, "race_workspace_size: bad args");
    *bytes = static_cast<size_t>(n_rows) * race_chunks(vocab) * sizeof(uint64_t);
    return NVS_OK;
}

extern "C" int nvs_race(const float* weights, int64_t weights_row_stride, const float* noise,
                        int64_t noise_row_stride, int64_t n_rows, int64_t vocab, int64_t* out,
                        int32_t* row_counters, void* workspace, size_t workspace_bytes, void* stream) {
    nvs::clear_error();
    NVS_CHECK(n_rows >= 0 && vocab > 0 && vocab < 0x7fffffffLL, NVS_ERR_INVALID, "race: bad sizes");
    NVS_CHECK(n_rows <= 0x7fffffffLL, NVS_ERR_UNSUPPORTED, "race: too many rows");
    if (n_rows == 0) return NVS_OK;
    NVS_CHECK(weights && noise && out && row_counters, NVS_ERR_INVALID, "race: null pointer");
    // stride 0 = one row broadcast over all rows (an expanded tensor)
    NVS_CHECK((weights_row_stride == 0 || weights_row_stride >= vocab) &&
                  (noise_row_stride == 0 || noise_row_stride >= vocab),
              NVS_ERR_INVALID, "race: bad row strides");
    size_t need = 0;
    nvs_race_workspace_size(n_rows, vocab, &need);
    NVS_CHECK(workspace != nullptr && workspace_bytes >= need, NVS_ERR_WORKSPACE,
              "race: workspace of %zu bytes needed, %zu given", need, workspace_bytes);
    RaceArgs a{};
    a.p = weights;
    a.p_stride = weights_row_stride;
    a.noise = noise;
    a.noise_stride = noise_row_stride;
    a.rows = n_rows;
    a.vocab = vocab;
    a.n_chunks = static_cast<int>(race_chunks(vocab));
    a.partial = static_cast<uint64_t*>(workspace);
    a.counters = row_counters;
    a.out = out;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const bool vec = vocab % 4 == 0 && nvs::aligned16(weights) && nvs::aligned16(noise) &&
                     weights_row_stride % 4 == 0 && noise_row_stride % 4 == 0;
    if (vec) {
        hipLaunchKernelGGL((race_chunk_kernel<false, true>), dim3(n_rows, a.n_chunks), dim3(256), 0, s, a);
    } else {
        hipLaunchKernelGGL((race_chunk_kernel<false, false>), dim3(n_rows, a.n_chunks), dim3(256), 0, s, a);
    }
    return nvs::check_launch("race chunk kernel");
}

extern "C" int nvs_accept_random_workspace_size(int64_t batch, int64_t vocab, size_t* bytes) {
    return nvs_race_workspace_size(batch, vocab, bytes);
}

static int accept_common_checks(const int64_t* drafts, int64_t batch, int num_drafts, int64_t n_pos, int64_t vocab,
                                int64_t* n_accept, int64_t* tail) {
    NVS_CHECK(batch >= 0 && num_drafts >= 1 && n_pos >= 0 && vocab > 0, NVS_ERR_INVALID,
              "accept: bad sizes batch=%lld k=%d n_pos=%lld vocab=%lld", (long long)batch, num_drafts,
              (long long)n_pos, (long long)vocab);
    NVS_CHECK(vocab < 0x7fffffffLL && batch <= 0x7fffffffLL, NVS_ERR_UNSUPPORTED, "accept: sizes too large");
    NVS_CHECK(batch == 0 || (drafts && n_accept && tail), NVS_ERR_INVALID, "accept: null pointer");
    return NVS_OK;
}

extern "C" int nvs_accept_random(const float* p, const float* q, const int64_t* drafts, const int64_t* verified_lens,
                                 const float* uniforms, const float* noise, int64_t batch, int num_drafts,
                                 int64_t n_pos, int64_t vocab, int64_t* n_accept, int64_t* tail,
                                 int32_t* row_counters, void* workspace, size_t workspace_bytes, void* stream) {
    nvs::clear_error();
    int st = accept_common_checks(drafts, batch, num_drafts, n_pos, vocab, n_accept, tail);
    if (st != NVS_OK) return st;
    if (batch == 0) return NVS_OK;
    NVS_CHECK(p && q && uniforms && noise && row_counters, NVS_ERR_INVALID, "accept_random: null pointer");
    NVS_CHECK(verified_lens != nullptr || n_pos == batch * (num_drafts + 1), NVS_ERR_INVALID,
              "accept_random: p has %lld positions, expected batch*(k+1) = %lld", (long long)n_pos,
              (long long)(batch * (num_drafts + 1)));
    size_t need = 0;
    nvs_race_workspace_size(batch, vocab, &need);
    NVS_CHECK(workspace != nullptr && workspace_bytes >= need, NVS_ERR_WORKSPACE,
              "accept_random: workspace of %zu bytes needed, %zu given", need, workspace_bytes);
    RaceArgs a{};
    a.p = p;
    a.p_stride = vocab;
    a.q = q;
    a.noise = noise;
    a.noise_stride = vocab;
    a.drafts = drafts;
    a.lens = verified_lens;
    a.uniforms = uniforms;
    a.rows = batch;
    a.n_pos = n_pos;
    a.k = num_drafts;
    a.vocab = vocab;
    a.n_chunks = static_cast<int>(race_chunks(vocab));
    a.partial = static_cast<uint64_t*>(workspace);
    a.counters = row_counters;
    a.n_accept = n_accept;
    a.out = tail;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const bool vec = vocab % 4 == 0 && nvs::aligned16(p) && nvs::aligned16(q) && nvs::aligned16(noise);
    if (vec) {
        hipLaunchKernelGGL((race_chunk_kernel<true, true>), dim3(batch, a.n_chunks), dim3(256), 0, s, a);
    } else {
        hipLaunchKernelGGL((race_chunk_kernel<true, false>), dim3(batch, a.n_chunks), dim3(256), 0, s, a);
    }
    return nvs::check_launch("accept_random chunk kernel");
}

extern "C" int nvs_accept_greedy_workspace_size(int64_t n_pos, int64_t vocab, size_t* bytes) {
    nvs::clear_error();
    (void)vocab;
    NVS_CHECK(bytes != nullptr && n_pos >= 0, NVS_ERR_INVALID, "accept_greedy_workspace_size: bad args");
    *bytes = static_cast<size_t>(n_pos) * sizeof(int64_t);
    return NVS_OK;
}

extern "C" int nvs_accept_greedy(const void* logits, int logits_dtype, int64_t logits_row_stride,
                                 const int64_t* drafts, const int64_t* verified_lens, int64_t batch, int num_drafts,
                                 int64_t n_pos, int64_t vocab, int64_t* n_accept, int64_t* tail, void* workspace,
                                 size_t workspace_bytes, void* stream) {
    nvs::clear_error();
    int st = check_dtype(logits_dtype);
    if (st != NVS_OK) return st;
    st = accept_common_checks(drafts, batch, num_drafts, n_pos, vocab, n_accept, tail);
    if (st != NVS_OK) return st;
    if (batch == 0) return NVS_OK;
    NVS_CHECK(logits != nullptr && logits_row_stride >= vocab, NVS_ERR_INVALID, "accept_greedy: bad logits");
    NVS_CHECK(verified_lens != nullptr || n_pos == batch * (num_drafts + 1), NVS_ERR_INVALID,
              "accept_greedy: logits have %lld positions, expected batch*(k+1) = %lld", (long long)n_pos,
              (long long)(batch * (num_drafts + 1)));
    NVS_CHECK(n_pos <= 0x7fffffffLL, NVS_ERR_UNSUPPORTED, "accept_greedy: too many positions");
    size_t need = static_cast<size_t>(n_pos) * sizeof(int64_t);
    NVS_CHECK(workspace != nullptr && workspace_bytes >= need, NVS_ERR_WORKSPACE,
              "accept_greedy: workspace of %zu bytes needed, %zu given", need, workspace_bytes);
    int64_t* tokens = static_cast<int64_t*>(workspace);
    hipStream_t s = static_cast<hipStream_t>(stream);
    switch (logits_dtype) {
        case NVS_DTYPE_F32: launch_argmax<NVS_DTYPE_F32>(logits, logits_row_stride, n_pos, vocab, tokens, s); break;
        case NVS_DTYPE_BF16: launch_argmax<NVS_DTYPE_BF16>(logits, logits_row_stride, n_pos, vocab, tokens, s); break;
        default: launch_argmax<NVS_DTYPE_F16>(logits, logits_row_stride, n_pos, vocab, tokens, s); break;
    }
    st = nvs::check_launch("accept_greedy argmax kernel");
    if (st != NVS_OK) return st;
    hipLaunchKernelGGL(greedy_finalize_kernel, dim3(static_cast<unsigned>(batch)), dim3(256), 0, s, tokens,
                       drafts, verified_lens, batch, n_pos, num_drafts, n_accept, tail);
    return nvs::check_launch("accept_greedy finalize kernel");
}

// Workspace of the fused accept: one 32-byte record per position (the per-row counters are a separate argument).
// ---------------------------------------------------------------- dense race of the fused accept
// Rows that do not truncate: the tail is argmax_i w_i / E_i over the whole vocabulary with p_i = exp(s_i - m) / Z
// recomputed from the tail position's logits (s = logit / temperature, NaN gives p = 0) and w = p for the bonus
// position, max(p - q, 0) otherwise: the same scores as the row finish's own loop, spread over (row, chunk)
// workgroups like the dense race kernels, then merged per row.

// Four consecutive logits of a row as floats: one 16-byte load (fp32) or one 8-byte load (16-bit).
template <int DT>
__device__ __forceinline__ float4 load4_as_float(const char* row, int64_t j) {
    if constexpr (DT == NVS_DTYPE_F32) {
        return reinterpret_cast<const float4*>(row)[j];
    } else {
        const uint2 w = reinterpret_cast<const uint2*>(row)[j];
        auto cv = [](uint32_t h) {
            if constexpr (DT == NVS_DTYPE_BF16) return nvs::bf16_bits_to_float(static_cast<uint16_t>(h));
            else return nvs::f16_bits_to_float(static_cast<uint16_t>(h));
        };
        return make_float4(cv(w.x & 0xffffu), cv(w.x >> 16), cv(w.y & 0xffffu), cv(w.y >> 16));
    }
}

template <int DT, bool VEC>
__global__ __launch_bounds__(256) void dense_race_chunk_kernel(SelArgs a) {
    __shared__ uint64_t red[4];
    const int64_t r = blockIdx.x;
    const int c = blockIdx.y;
    const DenseRace d = a.dense_race[r];
    if (!d.valid) return;   // the row's tail is its position's own race, already written (uniform per row)
    uint64_t best = 0;
    {
        const int64_t i0 = static_cast<int64_t>(c) * kRaceChunk;
        const int64_t i1 = min(i0 + kRaceChunk, a.vocab);
        const float* erow = a.noise + r * a.vocab;
        const char* row = static_cast<const char*>(a.logits) + d.pos * a.row_stride * nvs::dtype_size(DT);
        const bool bonus = d.qrow < 0;
        const float* qrow = a.q + (bonus ? 0 : d.qrow) * a.vocab;
        const float mu = (d.m == -INFINITY) ? 0.f : d.m;
        const bool unit_temp = (d.temp == 1.f);
        // sc: the logit already divided by the temperature (behind a uniform branch, not a select)
        auto key_of = [&](float sc, float q, float e, int64_t i) {
            const float p = (sc == sc) ? expf(sc - mu) / d.z : 0.f;
            const float w = bonus ? p : fmaxf(p - q, 0.f);
            const float score = w / e;
            return (static_cast<uint64_t>(nvs::float_key(score)) << 32) |
                   static_cast<uint64_t>(0xffffffffu - static_cast<uint32_t>(i));
        };
        if constexpr (VEC) {
            // every load first (noise, logits, q), from pieces clamped into the chunk
            float4 ev[kRacePer], xv[kRacePer], qv[kRacePer];
#pragma unroll
            for (int m = 0; m < kRacePer; ++m) {
                const int64_t j = min((i0 >> 2) + threadIdx.x + 256 * m, (i1 >> 2) - 1);
                ev[m] = reinterpret_cast<const float4*>(erow)[j];
                xv[m] = load4_as_float<DT>(row, j);
                qv[m] = reinterpret_cast<const float4*>(qrow)[j];
            }
            if (!unit_temp) {
#pragma unroll
                for (int m = 0; m < kRacePer; ++m) {
                    xv[m].x = xv[m].x / d.temp;
                    xv[m].y = xv[m].y / d.temp;
                    xv[m].z = xv[m].z / d.temp;
                    xv[m].w = xv[m].w / d.temp;
                }
            }
#pragma unroll
            for (int m = 0; m < kRacePer; ++m) {
                const int64_t j = (i0 >> 2) + threadIdx.x + 256 * m;
                if (j >= (i1 >> 2)) continue;
                const float x4[4] = {xv[m].x, xv[m].y, xv[m].z, xv[m].w};
                const float q4[4] = {qv[m].x, qv[m].y, qv[m].z, qv[m].w};
                const float e4[4] = {ev[m].x, ev[m].y, ev[m].z, ev[m].w};
#pragma unroll
                for (int l = 0; l < 4; ++l) {
                    const uint64_t k64 = key_of(x4[l], q4[l], e4[l], 4 * j + l);
                    best = best > k64 ? best : k64;
                }
            }
        } else {
            for (int64_t i = i0 + threadIdx.x; i < i1; i += blockDim.x) {
                const uint64_t k64 = key_of(scale_logit(nvs::load_as_float<DT>(row, i), d.temp, unit_temp),
                                            bonus ? 0.f : qrow[i], erow[i], i);
                best = best > k64 ? best : k64;
            }
        }
    }
    best = wave_max_u64(best);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = best;
    __syncthreads();
    if (threadIdx.x < 64) {
        // the row's counter was left at zero by the accept kernel's row finish; the row's last chunk writes the tail
        uint64_t all = 0;
        for (int w = 0; w < 4; ++w) all = red[w] > all ? red[w] : all;
        uint64_t win = 0;
        if (finish_race_chunk(a.dense_partial + r * a.dense_chunks, a.dense_chunks, c, all, a.counters + r, win) &&
            threadIdx.x == 0)
            a.tail[r] = static_cast<int64_t>(0xffffffffu - static_cast<uint32_t>(win));
    }
}

// Workspace of the fused accept: the position records, then (no truncating row) the dense races and their chunks.
struct AcceptLayout {
    size_t dense_off, partial_off, bytes;
};
AcceptLayout accept_layout(int64_t batch, int64_t n_pos, int64_t vocab, bool dense) {
    AcceptLayout l;
    l.bytes = static_cast<size_t>(n_pos) * sizeof(PosRecord);
    l.dense_off = l.partial_off = 0;
    if (dense) {
        l.dense_off = nvs::align_up(l.bytes, 256);
        l.partial_off = nvs::align_up(l.dense_off + static_cast<size_t>(batch) * sizeof(DenseRace), 256);
        l.bytes = l.partial_off + static_cast<size_t>(batch) * static_cast<size_t>(race_chunks(vocab)) * 8;
    }
    return l;
}

extern "C" int nvs_spec_accept_workspace_size(int64_t batch, int num_drafts, int64_t n_pos, int64_t vocab,
                                              int max_top_k, size_t* bytes) {
    nvs::clear_error();
    (void)num_drafts;
    NVS_CHECK(bytes != nullptr && n_pos >= 0 && batch >= 0 && vocab > 0, NVS_ERR_INVALID,
              "spec_accept_workspace_size: bad args");
    const int st = check_topk(max_top_k);
    if (st != NVS_OK) return st;
    *bytes = accept_layout(batch, n_pos, vocab, max_top_k == 0).bytes;
    return NVS_OK;
}

// The fused accept behind both entry points: q dense (q) or as candidate rows (q_ids / q_probs).
static int spec_accept_impl(const void* logits, int logits_dtype, int64_t logits_row_stride,
                            const float* temperatures, const int64_t* top_k, const float* top_p, int max_top_k,
                            int has_top_p, const float* q, const int32_t* q_ids, const float* q_probs, int q_cand,
                            int64_t q_stride, const int64_t* drafts, const int64_t* verified_lens,
                            const float* uniforms, const float* noise, int64_t batch, int num_drafts, int64_t n_pos,
                            int64_t vocab, int64_t* n_accept, int64_t* tail, int32_t* row_counters, void* workspace,
                            size_t workspace_bytes, void* stream) {
    int st = check_dtype(logits_dtype);
    if (st != NVS_OK) return st;
    st = accept_common_checks(drafts, batch, num_drafts, n_pos, vocab, n_accept, tail);
    if (st != NVS_OK) return st;
    st = common_select_checks(logits, logits_row_stride, n_pos, vocab, 1, max_top_k, top_k);
    if (st != NVS_OK) return st;
    if (batch == 0) return NVS_OK;
    NVS_CHECK(temperatures && (q || (q_ids && q_probs)) && uniforms && noise && row_counters, NVS_ERR_INVALID,
              "spec_accept: null pointer");
    NVS_CHECK(!has_top_p || top_p != nullptr, NVS_ERR_INVALID, "spec_accept: has_top_p needs top_p");
    NVS_CHECK(verified_lens != nullptr || n_pos == batch * (num_drafts + 1), NVS_ERR_INVALID,
              "spec_accept: logits have %lld positions, expected batch*(k+1) = %lld", (long long)n_pos,
              (long long)(batch * (num_drafts + 1)));
    // No row truncates (the reference's default sampling): each row's race over the whole vocabulary runs in
    // the dense race kernels after the accept kernel, spread over (row, chunk) workgroups.
    const bool dense = max_top_k == 0;
    const AcceptLayout lay = accept_layout(batch, n_pos, vocab, dense);
    NVS_CHECK(workspace != nullptr && workspace_bytes >= lay.bytes, NVS_ERR_WORKSPACE,
              "spec_accept: workspace of %zu bytes needed, %zu given", lay.bytes, workspace_bytes);
    SelArgs a{};
    a.logits = logits;
    a.row_stride = logits_row_stride;
    a.n_pos = n_pos;
    a.vocab = vocab;
    a.temps = temperatures;
    a.top_k = max_top_k > 0 ? top_k : nullptr;
    a.top_p = top_p;
    a.max_top_k = max_top_k;
    a.has_top_p = has_top_p && max_top_k > 0;
    a.pos_per_param = 1;
    a.q = q;
    a.q_ids = q_ids;
    a.q_probs = q_probs;
    a.q_cand = q_cand;
    a.q_stride = q_stride;
    a.drafts = drafts;
    a.lens = verified_lens;
    a.uniforms = uniforms;
    a.noise = noise;
    a.batch = batch;
    a.k = num_drafts;
    a.rec = static_cast<PosRecord*>(workspace);
    a.counters = row_counters;
    a.n_accept = n_accept;
    a.tail = tail;
    if (dense) {
        a.dense_race = reinterpret_cast<DenseRace*>(static_cast<char*>(workspace) + lay.dense_off);
        a.dense_partial = reinterpret_cast<uint64_t*>(static_cast<char*>(workspace) + lay.partial_off);
        a.dense_chunks = static_cast<int>(race_chunks(vocab));
    }
    hipStream_t s = static_cast<hipStream_t>(stream);
    st = launch_select<kModeAccept>(logits_dtype, a, s);
    if (st != NVS_OK || !dense) return st;
    const int es = nvs::dtype_size(logits_dtype);
    const bool vec = vocab % 4 == 0 && logits_row_stride % 4 == 0 && nvs::aligned16(noise) && nvs::aligned16(q) &&
                     (reinterpret_cast<uintptr_t>(logits) % (4 * es)) == 0;
    const dim3 grid(static_cast<unsigned>(batch), static_cast<unsigned>(a.dense_chunks));
    if (logits_dtype == NVS_DTYPE_F32) {
        if (vec) hipLaunchKernelGGL((dense_race_chunk_kernel<NVS_DTYPE_F32, true>), grid, dim3(256), 0, s, a);
        else hipLaunchKernelGGL((dense_race_chunk_kernel<NVS_DTYPE_F32, false>), grid, dim3(256), 0, s, a);
    } else if (logits_dtype == NVS_DTYPE_BF16) {
        if (vec) hipLaunchKernelGGL((dense_race_chunk_kernel<NVS_DTYPE_BF16, true>), grid, dim3(256), 0, s, a);
        else hipLaunchKernelGGL((dense_race_chunk_kernel<NVS_DTYPE_BF16, false>), grid, dim3(256), 0, s, a);
    } else {
        if (vec) hipLaunchKernelGGL((dense_race_chunk_kernel<NVS_DTYPE_F16, true>), grid, dim3(256), 0, s, a);
        else hipLaunchKernelGGL((dense_race_chunk_kernel<NVS_DTYPE_F16, false>), grid, dim3(256), 0, s, a);
    }
    return nvs::check_launch("spec_accept dense race");
}

namespace nvs {

size_t spec_accept_workspace_bytes(int64_t batch, int64_t n_pos, int64_t vocab, int max_top_k) {
    return accept_layout(batch, n_pos, vocab, max_top_k == 0).bytes;
}

int spec_accept_dense_q(const void* logits, int logits_dtype, int64_t logits_row_stride, const float* temperatures,
                        const int64_t* top_k, const float* top_p, int max_top_k, int has_top_p, const float* q,
                        const int64_t* drafts, const int64_t* verified_lens, const float* uniforms,
                        const float* noise, int64_t batch, int num_drafts, int64_t n_pos, int64_t vocab,
                        int64_t* n_accept, int64_t* tail, int32_t* row_counters, void* workspace,
                        size_t workspace_bytes, void* stream) {
    NVS_CHECK(q != nullptr || batch == 0, NVS_ERR_INVALID, "spec_accept: q is NULL");
    return spec_accept_impl(logits, logits_dtype, logits_row_stride, temperatures, top_k, top_p, max_top_k,
                            has_top_p, q, nullptr, nullptr, 0, 0, drafts, verified_lens, uniforms, noise, batch,
                            num_drafts, n_pos, vocab, n_accept, tail, row_counters, workspace, workspace_bytes,
                            stream);
}

}  // namespace nvs

extern "C" int nvs_spec_accept(const void* logits, int logits_dtype, int64_t logits_row_stride,
                               const float* temperatures, const int64_t* top_k, const float* top_p, int max_top_k,
                               int has_top_p, const float* q, const int64_t* drafts, const int64_t* verified_lens,
                               const float* uniforms, const float* noise, int64_t batch, int num_drafts,
                               int64_t n_pos, int64_t vocab, int64_t* n_accept, int64_t* tail,
                               int32_t* row_counters, void* workspace, size_t workspace_bytes, void* stream) {
    nvs::clear_error();
    return nvs::spec_accept_dense_q(logits, logits_dtype, logits_row_stride, temperatures, top_k, top_p, max_top_k,
                                    has_top_p, q, drafts, verified_lens, uniforms, noise, batch, num_drafts, n_pos,
                                    vocab, n_accept, tail, row_counters, workspace, workspace_bytes, stream);
}

extern "C" int nvs_spec_accept_candidates(const void* logits, int logits_dtype, int64_t logits_row_stride,
                                          const float* temperatures, const int64_t* top_k, const float* top_p,
                                          int max_top_k, int has_top_p, const int32_t* cand_ids,
                                          const float* cand_probs, int num_candidates, int64_t cand_row_stride,
                                          const int64_t* drafts, const int64_t* verified_lens, const float* uniforms,
                                          const float* noise, int64_t batch, int num_drafts, int64_t n_pos,
                                          int64_t vocab, int64_t* n_accept, int64_t* tail, int32_t* row_counters,
                                          void* workspace, size_t workspace_bytes, void* stream) {
    nvs::clear_error();
    NVS_CHECK(batch == 0 || (cand_ids != nullptr && cand_probs != nullptr), NVS_ERR_INVALID,
              "spec_accept_candidates: null candidate rows");
    NVS_CHECK(num_candidates >= 1 && cand_row_stride >= num_candidates, NVS_ERR_INVALID,
              "spec_accept_candidates: num_candidates %d with row stride %lld", num_candidates,
              (long long)cand_row_stride);
    NVS_CHECK(max_top_k >= 1, NVS_ERR_INVALID, "spec_accept_candidates: candidate rows need top-k (max_top_k >= 1)");
    return spec_accept_impl(logits, logits_dtype, logits_row_stride, temperatures, top_k, top_p, max_top_k,
                            has_top_p, nullptr, cand_ids, cand_probs, num_candidates, cand_row_stride, drafts,
                            verified_lens, uniforms, noise, batch, num_drafts, n_pos, vocab, n_accept, tail,
                            row_counters, workspace, workspace_bytes, stream);
}
