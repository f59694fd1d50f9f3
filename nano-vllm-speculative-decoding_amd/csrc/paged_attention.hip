// Paged multi-query verify attention for gfx950 (MI355X).
// Reference: Attention.forward, nanovllm/layers/attention.py:59-77 (flash_attn_varlen_func with block_table in the
// verify / cached-prefix branch, flash_attn_with_kvcache in the decode / draft-block branch); the semantics are
// restated in tests/fake_paged_attention.py:20-41 (gather through block_tables, GQA by head group, bottom-right
// causal rule j <= Lk - Lq + i).
//
// Work decomposition.
//   One workgroup = (request row r, kv head g, query tile qt, key split s); 4 wavefronts.
//   The query tile packs the GQA query heads of kv head g and all query positions of the row into 32 "packed rows"
//   n = qpos * group + hg, so every K/V byte of the row's kv head is read from HBM once for all of them
//   (Qwen3-8B: group 4 x 8 verify positions = 32 rows).
//   The key range [0, Lk) is cut into at most n_splits splits of equal size, whole 32-key chunks and at least
//   split_tokens keys each, sized from the row's own Lk on the device (the grid depends only on host integers, so
//   a captured graph serves every batch); each wave of the workgroup takes every 4th
//   32-key chunk of its split and keeps its own online-softmax state. The 4 waves are merged in LDS
//   (deterministic order); a row with a single split writes bf16 output directly, otherwise each split writes an
//   fp32 partial (O, max, sum) at the device's coherence point and counts itself on the unit's counter; the
//   unit's last split to finish merges every partial with the log-sum-exp rule, in split order (so the result
//   does not depend on which split finished last), and writes the bf16 output. One launch either way.
//
// Per chunk of 32 keys, per wave (lane l: packed row nl = l % 32, half gi = l / 32):
//   load    K and V rows of the chunk with coalesced streaming 16-byte loads (4 keys x 256 B per instruction,
//           page and block id clamped into range) and stage them into the wave's padded LDS tiles; the loads of
//           chunk c + 4 (the wave's next chunk) are issued right after, so they are in flight during the math
//   S^T[32 keys x 32 rows] = K[32 x 128] . Q^T      8 x v_mfma_f32_32x32x16_bf16 (_f16 for fp16 caches), K read from the LDS tile in the
//                                                    A-operand layout, Q from the LDS query tile
//   online softmax in fp32 with exp2 (scale * log2 e folded into one multiply); each lane owns one packed row,
//   the two halves of a row are merged with one cross-lane exchange
//   O^T[128 x 32] += V^T[128 x 32 keys] . P^T       8 x v_mfma_f32_32x32x16_bf16; P rounded to bf16 as the B
//                                                    operand straight from the S accumulators; V^T read from the
//                                                    [key][dim] LDS tile with transposing LDS loads
//                                                    (ds_read_b64_tr_b16, 2 per MFMA)
#include "nvs_common.hpp"

#include <cmath>

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef short tr_v4 __attribute__((ext_vector_type(4)));
typedef short tr_v8 __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) tr_v4 tr_lds;   // an LDS address of 4 bf16

// The two 16-bit element types the kernel serves (bf16, and fp16 for models built in half precision,
// model_runner.py:55-57): element, 8-element MFMA operand, the 32x32x16 MFMA and the fp32 -> 16-bit rounding
// (round to nearest even).
template <int DT> struct Elem16;
template <> struct Elem16<NVS_DTYPE_BF16> {
    typedef __bf16 type;
    typedef bf16x8 vec8;
    static __device__ __forceinline__ f32x16 mfma(vec8 a, vec8 b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
    }
    static __device__ __forceinline__ uint32_t bits(float f) { return nvs::float_to_bf16_bits(f); }
};
template <> struct Elem16<NVS_DTYPE_F16> {
    typedef _Float16 type;
    typedef f16x8 vec8;
    static __device__ __forceinline__ f32x16 mfma(vec8 a, vec8 b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
    }
    static __device__ __forceinline__ uint32_t bits(float f) { return __half_as_ushort(__float2half(f)); }
};

// Launch shape. kPrefetch: chunks of K/V each wave keeps in flight in registers (a ring, so the loads of the wave's
// next kPrefetch chunks are outstanding while one chunk is computed); kWgPerCu: resident workgroups per CU, which
// bounds the registers a wave may hold (256 at 2, 512 at 1).
#ifndef NVS_ATTN_PREFETCH
#define NVS_ATTN_PREFETCH 1
#endif
#ifndef NVS_ATTN_WG_PER_CU
#define NVS_ATTN_WG_PER_CU 2
#endif
#ifndef NVS_ATTN_ROWS_FIRST
#define NVS_ATTN_ROWS_FIRST 0
#endif
constexpr int kPrefetch = NVS_ATTN_PREFETCH;
constexpr int kWgPerCu = NVS_ATTN_WG_PER_CU;
// grid dimension order: (kv head x query tile, row, split), or with rows first (row, kv head x query tile, split)
constexpr bool kRowsFirst = NVS_ATTN_ROWS_FIRST != 0;

constexpr int kHeadDim = 128;
constexpr int kTileRows = 32;    // packed query rows per tile
constexpr int kChunk = 32;       // keys per MFMA chunk
constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kSplitQuantum = kChunk * kWaves;  // the planned split size is a multiple of this
// Wave-private K and V tiles in LDS: [32 keys][128 dims] bf16 each, rows padded from 256 to 272 B (68 dwords,
// 4 banks apart) so that the staging stores (8 lanes along one row), the K operand reads (32 rows at one column)
// and the transposed V reads (one row per half-wave, 32 consecutive dims) are all free of bank conflicts.
constexpr int kRowStride = kHeadDim + 8;                 // bf16 elements per staged row
constexpr int kTileElems = kChunk * kRowStride;          // one 32-key tile
constexpr int kWaveElems = 2 * kTileElems;               // K tile + V tile
constexpr int kObStride = 33;                            // fp32 per dim row of the cross-wave reduction buffer
static_assert(kWaves * kHeadDim * kObStride * 4 <= kWaves * kWaveElems * 2, "the waves' partials fit the tiles");
// A split's partial is staged in LDS over the reduction buffer: [32 rows][128 dims] fp32 (16-byte pieces swizzled
// by row), then the rows' (max, sum) pairs.
constexpr int kMaxSplits = 64;                           // the merge keeps [splits][32] (max, sum) pairs in LDS
// Query tile in LDS: [32 packed rows][128 dims] bf16 with the same padded rows (B-operand reads of 32 rows at one
// column per half-wave).
constexpr int kQsStride = kRowStride;

struct AttnArgs {
    const uint16_t* q;
    int64_t q_ts, q_hs;
    const uint16_t* kc;
    const uint16_t* vc;
    int64_t c_bs, c_ts, c_hs;
    const int32_t* bt;
    int64_t bt_rs;
    int bt_width;
    int64_t n_blocks;
    int64_t n_tokens;
    const int32_t* cu_q;
    const int32_t* cu_k;
    const int32_t* ctx;
    int q_fixed;
    int n_kv, group, block_size, causal;
    float scale_log2;
    uint16_t* out;
    int64_t o_ts, o_hs;
    float* part_o;   // [units, n_splits, 32, 128]
    float* part_ml;  // [units, n_splits, 32, 2]
    int* counters;   // [units] splits of the unit finished; zero between calls
    int n_splits, split_tokens, q_tiles;   // split_tokens: the smallest split of a row with several
};

struct RowInfo {
    int q0, lq, lk;
};

__device__ __forceinline__ RowInfo row_info(const AttnArgs& a, int r) {
    RowInfo ri;
    if (a.cu_q != nullptr) {
        ri.q0 = a.cu_q[r];
        ri.lq = a.cu_q[r + 1] - ri.q0;
        ri.lk = a.cu_k[r + 1] - a.cu_k[r];
    } else {
        ri.q0 = r * a.q_fixed;
        ri.lq = a.q_fixed;
        ri.lk = a.ctx[r];
    }
    return ri;
}

// Keys per split of a row with lk keys: the row cut into n = clamp(lk / min_tokens, 1, n_splits) equal splits
// (so each holds at least min_tokens keys when there are several), rounded up to whole 32-key chunks (a chunk
// never straddles a page). ceil(lk / that) <= n <= n_splits, so a length above max_seqlen_k cannot send the merge
// past the partial buffers.
__device__ __forceinline__ int row_split_tokens(int lk, int min_tokens, int n_splits) {
    if (n_splits <= 1) return max(lk, 1);
    const int n = max(1, min(n_splits, lk / min_tokens));
    const int even = (lk + n - 1) / n;
    return max((even + kChunk - 1) / kChunk * kChunk, kChunk);
}

// Splits holding keys of a row (at least one, so a row without keys still writes zeros).
__device__ __forceinline__ int active_splits(int lk, int split_len) {
    return lk > 0 ? (lk + split_len - 1) / split_len : 1;
}

__device__ __forceinline__ void compiler_fence() { asm volatile("" ::: "memory"); }

template <int DT>
__global__ __launch_bounds__(kThreads, kWgPerCu) void attn_split_kernel(AttnArgs a) {
    using E = Elem16<DT>;
    using V8 = typename E::vec8;
    __shared__ __attribute__((aligned(16))) uint16_t tiles[kWaves * kWaveElems];
    __shared__ __attribute__((aligned(16))) uint16_t qs[kTileRows * kQsStride];
    __shared__ float sm_m[kWaves][kTileRows];
    __shared__ float sm_l[kWaves][kTileRows];

    // grid (kv head x query tile, row, split): every unit's first split is dispatched before any second split, so
    // the idle splits of short rows (s >= the row's split count) sit at the end of the dispatch order
    const int r = kRowsFirst ? blockIdx.x : blockIdx.y;
    const int gq = kRowsFirst ? blockIdx.y : blockIdx.x;
    const int g = gq / a.q_tiles;
    const int qt = gq - g * a.q_tiles;
    const int s = blockIdx.z;
    const RowInfo ri = row_info(a, r);
    const int n_base = qt * kTileRows;
    if (ri.lq <= 0 || n_base >= a.group * ri.lq) return;
    const int split_len = row_split_tokens(ri.lk, a.split_tokens, a.n_splits);
    const int n_act = active_splits(ri.lk, split_len);
    if (s >= n_act) return;
    const int k0 = s * split_len;
    const int k1 = min(k0 + split_len, ri.lk);

    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int nl = lane & 31;
    const int gi = lane >> 5;
    const int32_t* btr = a.bt + static_cast<int64_t>(r) * a.bt_rs;
    // Coalesced loads: lane -> key 4i + lane/16 of the chunk, 16 B piece lane%16 of that key's 256 B head row.
    const int ld_key = lane >> 4;
    const int ld_piece = lane & 15;
    const int64_t head_off = static_cast<int64_t>(g) * a.c_hs + 8 * ld_piece;
    const int nch = (k1 - k0 + kChunk - 1) / kChunk;

    // The unit's block-table entries, one per lane (page k0 / block_size + lane), read once. A chunk takes its block
    // id with one readlane: a load there would put a memory round trip (about a microsecond under this stream) in
    // front of every chunk's K/V loads. A unit longer than 64 pages reads the table for the pages past them.
    const int page0 = k0 / a.block_size;
    const int bt_lane = btr[min(page0 + lane, a.bt_width - 1)];
    // Element offset of chunk c's first key in the cache (the same for K and V), the block id clamped into the cache.
    auto chunk_base = [&](int c) -> int64_t {
        const int tb = k0 + c * kChunk;
        const int page = min(tb / a.block_size, a.bt_width - 1);
        const int rel = page - page0;
        int64_t blk = static_cast<unsigned>(rel) < 64u ? __builtin_amdgcn_readlane(bt_lane, rel) : btr[page];
        blk = blk < 0 ? 0 : (blk >= a.n_blocks ? a.n_blocks - 1 : blk);
        const int in_page = tb - (tb / a.block_size) * a.block_size;
        return blk * a.c_bs + head_off + static_cast<int64_t>(in_page) * a.c_ts;
    };
    // Piece i of chunk c: key 4i + ld_key (clamped into [0, Lk) so a tail chunk never reads outside the row's pages;
    // a 32-key chunk never straddles a page because block_size is a multiple of 32), 16 B of K and of V.
    auto load_piece = [&](int c, int64_t base, int i, u32x4& kq, u32x4& vq) {
        const int tb = k0 + c * kChunk;
        const int t = min(tb + 4 * i + ld_key, ri.lk - 1);
        const int64_t off = base + static_cast<int64_t>(t - tb) * a.c_ts;
        // streaming (non-temporal) loads: every K/V byte is read exactly once, so keep it out of the caches' normal
        // replacement; measured ~15% more bandwidth than default loads on MI355X for this stream
        kq = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(a.kc + off));
        vq = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(a.vc + off));
    };
    auto load_chunk = [&](int c, u32x4 (&kr)[8], u32x4 (&vr)[8]) {
        const int64_t base = chunk_base(c);
#pragma unroll
        for (int i = 0; i < 8; ++i) load_piece(c, base, i, kr[i], vr[i]);
    };

    // This wave's first kPrefetch chunks are requested before the query tile, so they are in flight together.
    u32x4 kr[kPrefetch][8], vr[kPrefetch][8];
#pragma unroll
    for (int d = 0; d < kPrefetch; ++d)
        if (wave + kWaves * d < nch) load_chunk(wave + kWaves * d, kr[d], vr[d]);

    // The query tile -> LDS (zeros for packed rows past the row's Lq): 32 rows x 256 B, one 16 B piece per thread
    // and pass.
    for (int e = tid; e < kTileRows * (kHeadDim / 8); e += kThreads) {
        const int row = e >> 4;
        const int piece = e & 15;
        const int nn = n_base + row;
        const int qp = nn / a.group;
        u32x4 v = {0u, 0u, 0u, 0u};
        if (qp < ri.lq && ri.q0 + qp < a.n_tokens && ri.q0 + qp >= 0) {
            const int hh = g * a.group + (nn - qp * a.group);
            v = *reinterpret_cast<const u32x4*>(a.q + static_cast<int64_t>(ri.q0 + qp) * a.q_ts +
                                                static_cast<int64_t>(hh) * a.q_hs + 8 * piece);
        }
        *reinterpret_cast<u32x4*>(qs + row * kQsStride + 8 * piece) = v;
    }

    // This lane's packed query row.
    const int n = n_base + nl;
    const int qpos = n / a.group;
    const int hg = n - qpos * a.group;
    const bool qvalid = qpos < ri.lq && ri.q0 + qpos < a.n_tokens && ri.q0 + qpos >= 0;
    const int h = g * a.group + hg;
    // Last key this row may see inside the split (bottom-right causal alignment).
    int lim = (a.causal && qvalid) ? (ri.lk - ri.lq + qpos) : (ri.lk - 1);
    lim = min(lim, k1 - 1);

    uint16_t* ks = tiles + wave * kWaveElems;   // this wave's K tile
    uint16_t* vs = ks + kTileElems;             // and V tile
    // V^T operand through gfx950's transposing LDS load (ds_read_b64_tr_b16). Within each 16-lane group, lane i
    // receives element i % 4 of the 8-byte blocks addressed by lanes 4k + i / 4 (k = 0..3), as element k. Lane
    // 16g + 4k + q addresses key 4 (g / 2) + k, dims 16 (g % 2) + 4q .. + 3 of a 16-key, 32-dim slice of the
    // [key][dim] tile, so lane l receives keys 4 (l / 32) + 0..3 of dim l % 32: the A-operand run the P^T
    // operand's key order needs (two loads per MFMA: keys +0 and +8).
    __attribute__((address_space(3))) uint16_t* vs_l = (__attribute__((address_space(3))) uint16_t*)vs;
    const int tr_off = (4 * (lane >> 5) + ((lane >> 2) & 3)) * kRowStride + 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
    const uint16_t* qrow = qs + nl * kQsStride + 8 * gi;

    float m_run = -INFINITY;
    float l_run = 0.f;
    f32x16 o[4];
#pragma unroll
    for (int db = 0; db < 4; ++db) o[db] = f32x16{};
    // Registers -> the wave-private tiles, each register pair refilled with piece i of chunk cn (when cn < nch) as
    // soon as it is stored, so the next chunk's loads leave while the rest is still being stored. LDS executes one
    // wave's accesses in issue order; the fences keep the compiler from moving these stores above the previous
    // chunk's reads.
    auto stage_chunk = [&](u32x4 (&kr)[8], u32x4 (&vr)[8], int cn) {
        if (cn < nch) {
            const int64_t nbase = chunk_base(cn);
            compiler_fence();
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int row = 4 * i + ld_key;
                *reinterpret_cast<u32x4*>(ks + row * kRowStride + 8 * ld_piece) = kr[i];
                *reinterpret_cast<u32x4*>(vs + row * kRowStride + 8 * ld_piece) = vr[i];
                load_piece(cn, nbase, i, kr[i], vr[i]);
            }
            compiler_fence();
        } else {
            compiler_fence();
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int row = 4 * i + ld_key;
                *reinterpret_cast<u32x4*>(ks + row * kRowStride + 8 * ld_piece) = kr[i];
                *reinterpret_cast<u32x4*>(vs + row * kRowStride + 8 * ld_piece) = vr[i];
            }
            compiler_fence();
        }
    };

    // One chunk: stage it while requesting the chunk this wave does next, S^T = K Q^T, online softmax,
    // O^T += V^T P^T.
    auto process_chunk = [&](int c, u32x4 (&kr)[8], u32x4 (&vr)[8]) {
        const int tb = k0 + c * kChunk;
        stage_chunk(kr, vr, c + kWaves * kPrefetch);

        f32x16 acc = f32x16{};
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const V8 kb = __builtin_bit_cast(V8, *reinterpret_cast<const u32x4*>(ks + nl * kRowStride + 16 * i +
                                                                                  8 * gi));
            const V8 qb = __builtin_bit_cast(V8, *reinterpret_cast<const u32x4*>(qrow + 16 * i));
            acc = E::mfma(kb, qb, acc);
        }
        float mx = -INFINITY;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const int t = tb + 8 * (j >> 2) + 4 * gi + (j & 3);
            acc[j] = (t <= lim) ? acc[j] * a.scale_log2 : -INFINITY;
            mx = fmaxf(mx, acc[j]);
        }
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        const float m_new = fmaxf(m_run, mx);
        const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
        const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
        float ps = 0.f;
        V8 pb[2];
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const float pj = __builtin_amdgcn_exp2f(acc[j] - m_use);
            ps += pj;
            pb[j >> 3][j & 7] = static_cast<typename E::type>(pj);
        }
        l_run = l_run * alpha + ps;
        m_run = m_new;
#pragma unroll
        for (int db = 0; db < 4; ++db) o[db] *= alpha;

        // V^T operand: lane (dim 32db + nl, half gi) gathers keys 16hh + 8a + 4gi + b (a = 0, 1; b = 0..3), the
        // keys whose P values it holds in pb[hh], from the [key][dim] tile.
#pragma unroll
        for (int db = 0; db < 4; ++db) {
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                const tr_lds* p0 = (const tr_lds*)(vs_l + tr_off + 16 * hh * kRowStride + 32 * db);
                const tr_lds* p1 = (const tr_lds*)(vs_l + tr_off + (16 * hh + 8) * kRowStride + 32 * db);
                const tr_v4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(const_cast<tr_lds*>(p0));
                const tr_v4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(const_cast<tr_lds*>(p1));
                const tr_v8 v8 = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                o[db] = E::mfma(__builtin_bit_cast(V8, v8), pb[hh], o[db]);
            }
        }
    };

    __syncthreads();  // query tile staged

    // This wave's chunks are wave, wave + 4, ...; chunk c sits in ring slot (c / 4) % kPrefetch, and its slot is
    // refilled with chunk c + 4 kPrefetch as soon as c is staged. The ring is unrolled so its slots stay registers.
    for (int c0 = wave; c0 < nch; c0 += kWaves * kPrefetch) {
#pragma unroll
        for (int d = 0; d < kPrefetch; ++d) {
            const int c = c0 + kWaves * d;
            if (c < nch) process_chunk(c, kr[d], vr[d]);
        }
    }

    // ---- merge the 4 waves (fixed order, so the result does not depend on timing)
    const float l_tot = l_run + __shfl_xor(l_run, 32);
    if (gi == 0) {
        sm_m[wave][nl] = m_run;
        sm_l[wave][nl] = l_tot;
    }
    __syncthreads();
    float mw[kWaves];
    float m_all = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
        mw[w] = sm_m[w][nl];
        m_all = fmaxf(m_all, mw[w]);
    }
    const float m_all_use = (m_all == -INFINITY) ? 0.f : m_all;
    float l_all = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) l_all += sm_l[w][nl] * __builtin_amdgcn_exp2f(mw[w] - m_all_use);
    const float own = __builtin_amdgcn_exp2f(m_run - m_all_use);
#pragma unroll
    for (int db = 0; db < 4; ++db) o[db] *= own;

    // Every wave stages its scaled partial O in LDS ([wave][dim][row], the K/V tiles are dead after the barrier
    // above); then wave w sums the four partials of dims 32w .. 32w + 31, in wave order (so the result does not
    // depend on timing), into the register layout o[w] had. One barrier instead of four sequential passes.
    float* ob = reinterpret_cast<float*>(tiles);
#pragma unroll
    for (int db = 0; db < 4; ++db) {
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const int d = 32 * db + 8 * (j >> 2) + 4 * gi + (j & 3);
            ob[(wave * kHeadDim + d) * kObStride + nl] = o[db][j];
        }
    }
    __syncthreads();
    f32x16 osum;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        const int d = 32 * wave + 8 * (j >> 2) + 4 * gi + (j & 3);
        float v = ob[d * kObStride + nl];
#pragma unroll
        for (int w = 1; w < kWaves; ++w) v += ob[(w * kHeadDim + d) * kObStride + nl];
        osum[j] = v;
    }
    if (n_act == 1) {
        if (!qvalid) return;
        const float inv = l_all > 0.f ? 1.f / l_all : 0.f;
        uint16_t* op = a.out + static_cast<int64_t>(ri.q0 + qpos) * a.o_ts + static_cast<int64_t>(h) * a.o_hs;
#pragma unroll
        for (int jq = 0; jq < 4; ++jq) {
            const int d = 32 * wave + 8 * jq + 4 * gi;
            const uint32_t lo = E::bits(osum[4 * jq + 0] * inv) | (E::bits(osum[4 * jq + 1] * inv) << 16);
            const uint32_t hi = E::bits(osum[4 * jq + 2] * inv) | (E::bits(osum[4 * jq + 3] * inv) << 16);
            *reinterpret_cast<u32x2*>(op + d) = u32x2{lo, hi};
        }
        return;
    }

    // Several splits. The partial (fp32 O and the per-row max and sum) is staged in LDS as [32 rows][128 dims] and
    // written to the coherence point with device-scope stores, 512 contiguous bytes per wave instruction, so the
    // unit's last split to finish reads it from any XCD.
    const int64_t unit = (static_cast<int64_t>(r) * a.n_kv + g) * a.q_tiles + qt;
    const int64_t pidx = unit * a.n_splits + s;
    float* stage = reinterpret_cast<float*>(tiles);   // over the partials just read
    float2* stage_ml = reinterpret_cast<float2*>(stage + kTileRows * kHeadDim);
    __syncthreads();   // every wave has read the staged partials before the stage overwrites them
#pragma unroll
    for (int jq = 0; jq < 4; ++jq) {
        const int d = 32 * wave + 8 * jq + 4 * gi;
        *reinterpret_cast<float4*>(stage + nl * kHeadDim + (d ^ ((nl & 7) << 2))) =
            make_float4(osum[4 * jq], osum[4 * jq + 1], osum[4 * jq + 2], osum[4 * jq + 3]);
    }
    if (wave == 0 && gi == 0) stage_ml[nl] = make_float2(m_all, l_all);
    __syncthreads();
    {
        uint64_t* po = reinterpret_cast<uint64_t*>(a.part_o + pidx * kTileRows * kHeadDim);
#pragma unroll
        for (int k = 0; k < kTileRows * kHeadDim / 2 / kThreads; ++k) {
            const int e = tid + kThreads * k;          // u64 element of the [32][128] fp32 partial
            const int row = e >> 6;
            const int d = 2 * (e & 63);
            const float2 v = *reinterpret_cast<const float2*>(stage + row * kHeadDim + (d ^ ((row & 7) << 2)));
            __hip_atomic_store(po + e, static_cast<uint64_t>(__float_as_uint(v.x)) |
                                           (static_cast<uint64_t>(__float_as_uint(v.y)) << 32),
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        if (tid < kTileRows) {
            const float2 v = stage_ml[tid];
            __hip_atomic_store(reinterpret_cast<uint64_t*>(a.part_ml) + pidx * kTileRows + tid,
                               static_cast<uint64_t>(__float_as_uint(v.x)) |
                                   (static_cast<uint64_t>(__float_as_uint(v.y)) << 32),
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    // vmcnt(0) in every wave: all of the workgroup's partial stores have completed before the count
    __builtin_amdgcn_s_waitcnt(0x0F70);
    __shared__ int last_split;
    __syncthreads();
    if (tid == 0) {
        const int before = __hip_atomic_fetch_add(a.counters + unit, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        last_split = (before == n_act - 1) ? 1 : 0;
    }
    __syncthreads();
    if (!last_split) return;

    // The unit's last split merges all n_act partials in split order (the result does not depend on which split
    // finished last). Every load is issued after this workgroup's own count returned, at the coherence point.
    if (tid == 0) __hip_atomic_store(a.counters + unit, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    float2* ml = reinterpret_cast<float2*>(tiles);           // [n_act][32] (max, sum), then the split weights
    float* inv_l = reinterpret_cast<float*>(ml + kMaxSplits * kTileRows);
    const uint64_t* pml = reinterpret_cast<const uint64_t*>(a.part_ml) + unit * a.n_splits * kTileRows;
    for (int e = tid; e < n_act * kTileRows; e += kThreads) {
        const uint64_t v = __hip_atomic_load(pml + e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        ml[e] = make_float2(__uint_as_float(static_cast<uint32_t>(v)), __uint_as_float(static_cast<uint32_t>(v >> 32)));
    }
    __syncthreads();
    if (tid < kTileRows) {
        float m_u = -INFINITY;
        for (int sp = 0; sp < n_act; ++sp) m_u = fmaxf(m_u, ml[sp * kTileRows + tid].x);
        const float m_uu = (m_u == -INFINITY) ? 0.f : m_u;
        float l_u = 0.f;
        for (int sp = 0; sp < n_act; ++sp) {
            const float w = __builtin_amdgcn_exp2f(ml[sp * kTileRows + tid].x - m_uu);
            l_u += ml[sp * kTileRows + tid].y * w;
            ml[sp * kTileRows + tid].x = w;   // the split's weight for this row
        }
        inv_l[tid] = l_u > 0.f ? 1.f / l_u : 0.f;
    }
    __syncthreads();
    // thread -> u64 elements tid + 256 k (k < 8) of the [32][128] partials: rows tid / 64 + 4 k, dims 2 (tid % 64)
    constexpr int kPer = kTileRows * kHeadDim / 2 / kThreads;
    float acc[kPer][2];
#pragma unroll
    for (int k = 0; k < kPer; ++k) acc[k][0] = acc[k][1] = 0.f;
    const uint64_t* pu = reinterpret_cast<const uint64_t*>(a.part_o) + unit * a.n_splits * kTileRows * kHeadDim / 2;
    for (int sp = 0; sp < n_act; ++sp) {
        uint64_t v[kPer];
#pragma unroll
        for (int k = 0; k < kPer; ++k)
            v[k] = __hip_atomic_load(pu + sp * (kTileRows * kHeadDim / 2) + tid + kThreads * k, __ATOMIC_RELAXED,
                                     __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
        for (int k = 0; k < kPer; ++k) {
            const float w = ml[sp * kTileRows + (tid >> 6) + 4 * k].x;
            acc[k][0] += __uint_as_float(static_cast<uint32_t>(v[k])) * w;
            acc[k][1] += __uint_as_float(static_cast<uint32_t>(v[k] >> 32)) * w;
        }
    }
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
        const int row = (tid >> 6) + 4 * k;
        const int nm = n_base + row;
        const int qpm = nm / a.group;
        if (qpm >= ri.lq || ri.q0 + qpm >= a.n_tokens || ri.q0 + qpm < 0) continue;
        const int hm = g * a.group + (nm - qpm * a.group);
        const float inv = inv_l[row];
        const uint32_t bits = E::bits(acc[k][0] * inv) | (E::bits(acc[k][1] * inv) << 16);
        *reinterpret_cast<uint32_t*>(a.out + static_cast<int64_t>(ri.q0 + qpm) * a.o_ts +
                                     static_cast<int64_t>(hm) * a.o_hs + 2 * (tid & 63)) = bits;
    }
}

struct SplitPlan {
    int q_tiles, n_splits, split_tokens;
    size_t workspace;
};

// Key-split plan: enough workgroups to fill the 256 CUs a few times over, each wave still streaming several
// chunks. Depends only on host integers, so it is stable under graph capture.
SplitPlan plan_splits(int n_rows, int n_heads, int n_kv_heads, int max_seqlen_q, int max_seqlen_k) {
    SplitPlan p;
    const int group = n_heads / n_kv_heads;
    p.q_tiles = (group * max_seqlen_q + kTileRows - 1) / kTileRows;
    const int64_t units = static_cast<int64_t>(n_rows) * n_kv_heads * p.q_tiles;
    // One resident round of workgroups: 256 CUs x 2 workgroups (the kernel's occupancy). Keys are split only when
    // the (row, kv head, tile) units fill less than half of that round, and then into enough splits to fill it:
    // measured on batch-8/16/32 verify layers (3k contexts), a split costs its partial and the merge, which a grid
    // of one unsplit workgroup per CU does not win back, while a grid under one workgroup per CU does.
    constexpr int64_t kRound = 256 * kWgPerCu;
    int64_t want = 1;
    if (units > 0 && units * 2 < kRound) want = (kRound + units - 1) / units;
    const int64_t max_k = max_seqlen_k > 0 ? max_seqlen_k : 1;
    int64_t ts = (max_k + want - 1) / want;
    int64_t min_ts = 2 * kSplitQuantum;   // a row's split holds at least this many keys (the device sizes them)
    if (ts * kMaxSplits < max_k) ts = (max_k + kMaxSplits - 1) / kMaxSplits;   // at most kMaxSplits splits
    ts = (ts + kSplitQuantum - 1) / kSplitQuantum * kSplitQuantum;
    if (ts < min_ts) ts = min_ts;
    // The grid has n_splits splits per unit, from max_seqlen_k; each row spreads its own keys over them on the
    // device, at least split_tokens per split.
    p.split_tokens = static_cast<int>(min_ts);
    p.n_splits = static_cast<int>((max_k + ts - 1) / ts);
    if (p.n_splits < 1) p.n_splits = 1;
    p.workspace = 0;
    if (p.n_splits > 1) {
        const size_t per = static_cast<size_t>(kTileRows) * (kHeadDim + 2) * sizeof(float);
        p.workspace = static_cast<size_t>(units) * p.n_splits * per + 256;
    }
    return p;
}

int validate_sizes(int n_rows, int n_heads, int n_kv_heads, int head_dim, int max_seqlen_q, int max_seqlen_k) {
    NVS_CHECK(n_rows >= 0 && max_seqlen_q >= 0 && max_seqlen_k >= 0, NVS_ERR_INVALID,
              "paged_attention: negative size (n_rows=%d max_seqlen_q=%d max_seqlen_k=%d)", n_rows, max_seqlen_q,
              max_seqlen_k);
    NVS_CHECK(n_heads > 0 && n_kv_heads > 0 && n_heads % n_kv_heads == 0, NVS_ERR_INVALID,
              "paged_attention: n_heads=%d must be a positive multiple of n_kv_heads=%d", n_heads, n_kv_heads);
    NVS_CHECK(head_dim == kHeadDim, NVS_ERR_UNSUPPORTED, "paged_attention: head_dim %d unsupported (only 128)",
              head_dim);
    return NVS_OK;
}

}  // namespace

extern "C" int nvs_paged_attention_workspace_size(int n_rows, int n_heads, int n_kv_heads, int head_dim,
                                                  int max_seqlen_q, int max_seqlen_k, size_t* bytes) {
    nvs::clear_error();
    NVS_CHECK(bytes != nullptr, NVS_ERR_INVALID, "paged_attention_workspace_size: bytes is NULL");
    const int st = validate_sizes(n_rows, n_heads, n_kv_heads, head_dim, max_seqlen_q, max_seqlen_k);
    if (st != NVS_OK) return st;
    *bytes = plan_splits(n_rows, n_heads, n_kv_heads, max_seqlen_q, max_seqlen_k).workspace;
    return NVS_OK;
}

extern "C" int nvs_paged_attention(const void* q, int64_t q_token_stride, int64_t q_head_stride, int64_t n_tokens,
                                   const void* k_cache, const void* v_cache, int64_t cache_blocks,
                                   int64_t cache_block_stride, int64_t cache_token_stride,
                                   int64_t cache_head_stride, const int32_t* block_tables, int64_t bt_row_stride,
                                   int bt_width, const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                                   const int32_t* context_lens, int query_len_per_seq, int n_rows, int max_seqlen_q,
                                   int max_seqlen_k, int n_heads, int n_kv_heads, int head_dim, int block_size,
                                   float scale, int causal, int dtype, void* out, int64_t out_token_stride,
                                   int64_t out_head_stride, int32_t* unit_counters, void* workspace,
                                   size_t workspace_bytes, void* stream) {
    nvs::clear_error();
    int st = validate_sizes(n_rows, n_heads, n_kv_heads, head_dim, max_seqlen_q, max_seqlen_k);
    if (st != NVS_OK) return st;
    NVS_CHECK(dtype == NVS_DTYPE_BF16 || dtype == NVS_DTYPE_F16, NVS_ERR_UNSUPPORTED,
              "paged_attention: dtype %d unsupported (bf16 or fp16)", dtype);
    const bool varlen = cu_seqlens_q != nullptr || cu_seqlens_k != nullptr;
    NVS_CHECK(!varlen || (cu_seqlens_q != nullptr && cu_seqlens_k != nullptr), NVS_ERR_INVALID,
              "paged_attention: cu_seqlens_q and cu_seqlens_k must both be given (varlen) or both NULL");
    NVS_CHECK(varlen || context_lens != nullptr, NVS_ERR_INVALID,
              "paged_attention: fixed mode needs context_lens");
    NVS_CHECK(varlen || query_len_per_seq >= 1, NVS_ERR_INVALID,
              "paged_attention: query_len_per_seq must be >= 1, got %d", query_len_per_seq);
    NVS_CHECK(varlen || query_len_per_seq <= max_seqlen_q, NVS_ERR_INVALID,
              "paged_attention: query_len_per_seq %d exceeds max_seqlen_q %d", query_len_per_seq, max_seqlen_q);
    NVS_CHECK(block_size > 0 && block_size % kChunk == 0, NVS_ERR_UNSUPPORTED,
              "paged_attention: block_size %d must be a positive multiple of %d", block_size, kChunk);
    if (n_rows == 0 || max_seqlen_q == 0 || n_tokens == 0) return NVS_OK;
    NVS_CHECK(n_tokens > 0 && cache_blocks > 0 && bt_width > 0, NVS_ERR_INVALID,
              "paged_attention: n_tokens=%lld, cache_blocks=%lld and bt_width=%d must be positive",
              (long long)n_tokens, (long long)cache_blocks, bt_width);
    NVS_CHECK(q && k_cache && v_cache && block_tables && out, NVS_ERR_INVALID, "paged_attention: null pointer");
    NVS_CHECK(nvs::aligned16(q) && nvs::aligned16(k_cache) && nvs::aligned16(v_cache), NVS_ERR_INVALID,
              "paged_attention: q, k_cache and v_cache must be 16-byte aligned");
    NVS_CHECK(q_token_stride % 8 == 0 && q_head_stride % 8 == 0 && cache_block_stride % 8 == 0 &&
                  cache_token_stride % 8 == 0 && cache_head_stride % 8 == 0,
              NVS_ERR_INVALID, "paged_attention: q and cache strides must be multiples of 8 elements");
    NVS_CHECK((reinterpret_cast<uintptr_t>(out) & 7u) == 0 && out_token_stride % 4 == 0 && out_head_stride % 4 == 0,
              NVS_ERR_INVALID, "paged_attention: out must be 8-byte aligned with strides multiple of 4");
    NVS_CHECK(scale > 0.f && std::isfinite(scale), NVS_ERR_INVALID, "paged_attention: bad scale %g", (double)scale);

    const SplitPlan plan = plan_splits(n_rows, n_heads, n_kv_heads, max_seqlen_q, max_seqlen_k);
    NVS_CHECK(plan.workspace == 0 || (workspace != nullptr && workspace_bytes >= plan.workspace),
              NVS_ERR_WORKSPACE, "paged_attention: workspace of %zu bytes needed, %zu given", plan.workspace,
              workspace_bytes);
    NVS_CHECK(plan.n_splits == 1 || unit_counters != nullptr, NVS_ERR_INVALID,
              "paged_attention: this plan splits keys and needs unit_counters");
    NVS_CHECK(static_cast<int64_t>(n_kv_heads) * plan.q_tiles <= 65535 && n_rows <= 65535, NVS_ERR_UNSUPPORTED,
              "paged_attention: grid too large (rows %d, kv heads x tiles %lld)", n_rows,
              (long long)n_kv_heads * plan.q_tiles);

    AttnArgs a;
    a.q = static_cast<const uint16_t*>(q);
    a.q_ts = q_token_stride;
    a.q_hs = q_head_stride;
    a.kc = static_cast<const uint16_t*>(k_cache);
    a.vc = static_cast<const uint16_t*>(v_cache);
    a.c_bs = cache_block_stride;
    a.c_ts = cache_token_stride;
    a.c_hs = cache_head_stride;
    a.bt = block_tables;
    a.bt_rs = bt_row_stride;
    a.bt_width = bt_width;
    a.n_blocks = cache_blocks;
    a.n_tokens = n_tokens;
    a.cu_q = varlen ? cu_seqlens_q : nullptr;
    a.cu_k = varlen ? cu_seqlens_k : nullptr;
    a.ctx = varlen ? nullptr : context_lens;
    a.q_fixed = varlen ? 0 : query_len_per_seq;
    a.n_kv = n_kv_heads;
    a.group = n_heads / n_kv_heads;
    a.block_size = block_size;
    a.causal = causal ? 1 : 0;
    a.scale_log2 = scale * 1.4426950408889634f;
    a.out = static_cast<uint16_t*>(out);
    a.o_ts = out_token_stride;
    a.o_hs = out_head_stride;
    char* ws = static_cast<char*>(workspace);
    const size_t po_bytes = plan.n_splits > 1 ? nvs::align_up(static_cast<size_t>(n_rows) * n_kv_heads *
                                                                   plan.q_tiles * plan.n_splits * kTileRows *
                                                                   kHeadDim * sizeof(float),
                                                               256)
                                              : 0;
    a.part_o = plan.n_splits > 1 ? reinterpret_cast<float*>(ws) : nullptr;
    a.part_ml = plan.n_splits > 1 ? reinterpret_cast<float*>(ws + po_bytes) : nullptr;
    a.counters = unit_counters;
    a.n_splits = plan.n_splits;
    a.split_tokens = plan.split_tokens;
    a.q_tiles = plan.q_tiles;

    hipStream_t s = static_cast<hipStream_t>(stream);
    const dim3 grid = kRowsFirst ? dim3(n_rows, n_kv_heads * plan.q_tiles, plan.n_splits)
                                 : dim3(n_kv_heads * plan.q_tiles, n_rows, plan.n_splits);
    if (dtype == NVS_DTYPE_BF16) {
        hipLaunchKernelGGL(attn_split_kernel<NVS_DTYPE_BF16>, grid, dim3(kThreads), 0, s, a);
    } else {
        hipLaunchKernelGGL(attn_split_kernel<NVS_DTYPE_F16>, grid, dim3(kThreads), 0, s, a);
    }
    return nvs::check_launch("paged_attention split kernel");
}
