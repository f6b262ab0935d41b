// attention.hip -- AttentionKernelOp: paged decode on bf16 MFMA, plus a
// general kernel for dense K/V, fp32 and uncommon shapes.
//
// Semantics: src/core/TensorCalc.cpp:1167-1314 (attention_impl).  Query qi of
// batch b sits at position offsets[b] + qi; key ki attends when
// ki <= position and (window == 0 or ki > position - window); scores are
// (q . k) * scale with scale <= 0 meaning 1/sqrt(D); softmax over the keys;
// an all-masked row gives zeros; GQA maps q head h to kv head h / (Hq/Hkv).
//
// Paged decode (the hot path).  The reference runs one
// 32-lane warp per (split, q head, batch): every q head re-reads its KV head
// (8x redundant for TinyLlama), with scalar fp32 FMAs, per-element paged
// address math and a cudaMallocAsync of the split partials on every call
// (CudaAttentionKernels.cu:247-404,469-563).  Here one 256-thread workgroup
// owns (split of keys, kv head, sequence) and the whole GQA group of q heads:
//   - K tiles of 16 keys are read from their page with 128-bit loads straight
//     into MFMA A operands; S^T = K Q^T on v_mfma_f32_16x16x32_bf16 (the head
//     group padded to 16 columns);
//   - online softmax in the exp2 domain, per q head (one MFMA column);
//   - P^T leaves the S^T MFMA already in the B-operand layout of
//     v_mfma_f32_16x16x16_bf16, and V tiles are transposed through LDS into A
//     operands, so O^T += V^T P^T runs on MFMA with no register shuffles;
//   - block ids, Q and the position are fetched together; each wave keeps
//     two batches of tiles in flight (ping-pong) while computing;
//   - the 4 waves merge in LDS and every split slot writes a (max, sum,
//     O[D]) partial to a persistent workspace (empty slots write max = -inf);
//     a small second kernel merges the slots (log-sum-exp) with one round of
//     loads.  No host round trip and no allocation per call.
// The probabilities fed to the PV product are rounded to bf16 and the
// normaliser sums those rounded values, so O / L stays a convex combination.
#include "common.h"

#include <algorithm>
#include <cstdlib>

namespace sandy_hip {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef short short4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;

struct PagedArgs {
    const uint16_t* q;
    int64_t q_sb, q_sh;  // element strides of q over batch and head (last dim contiguous)
    uint16_t* out;
    int64_t o_sb, o_sh;
    const uint16_t* k_pool;
    const uint16_t* v_pool;
    int64_t page_elems;  // Hkv * P * D
    int64_t num_pages;
    const int32_t* table;
    int64_t table_stride;
    int64_t max_blocks;
    const void* pos;
    int32_t pos_dt;
    int32_t page_size;
    int32_t log2_page;
    int32_t hq, hkv, group;
    int64_t window;
    float scale_log2;  // scale * log2(e)
    int32_t split_keys;
    int32_t max_splits;
    float* ws_o;   // [B, Hq, max_splits, D]
    float* ws_ml;  // [B, Hq, max_splits, 2]
    uint32_t* errw;
    uint32_t* counters;  // [B, Hkv] arrival counts of the fused merge
    int32_t fused_merge;
};

__device__ __forceinline__ short4_t pack_p(const float (&p)[4]) {
    short4_t r;
#pragma unroll
    for (int i = 0; i < 4; i++) r[i] = static_cast<short>(f32_to_bf16(p[i]));
    return r;
}

template <int D>
struct TileRegs {
    uint4 k[D / 32];
    uint4 v[D / 32];
};

// Loads one 16-key tile of K and V (this lane: key lane%16, 8 dims per MFMA
// k-step) from block `blk` (already validated; -1 = skip).
template <int D>
__device__ __forceinline__ void load_tile(const PagedArgs& a, int64_t t0, int32_t blk, int kh, int lane,
                                          TileRegs<D>& r) {
    const int64_t safe = blk < 0 ? 0 : blk;
    const int64_t in_page = t0 & (a.page_size - 1);
    const int64_t row = safe * a.page_elems + static_cast<int64_t>(kh) * a.page_size * D +
                        (in_page + (lane & 15)) * D + 8 * (lane >> 4);
    const uint4* kp = reinterpret_cast<const uint4*>(a.k_pool + row);
    const uint4* vp = reinterpret_cast<const uint4*>(a.v_pool + row);
#pragma unroll
    for (int kk = 0; kk < D / 32; kk++) {
        r.k[kk] = kp[kk * 4];  // + 32 elements per step
        r.v[kk] = vp[kk * 4];
    }
}

// Key range of one split of sequence b; shared by the attention and merge kernels.
struct SplitRange {
    int64_t n_keys, min_key, key_begin;
    int n_splits;
};

__device__ __forceinline__ SplitRange split_range(const PagedArgs& a, int64_t pos) {
    SplitRange r;
    r.n_keys = min(pos + 1, a.max_blocks * static_cast<int64_t>(a.page_size));
    r.min_key = a.window > 0 ? max<int64_t>(0, pos + 1 - a.window) : 0;
    r.key_begin = (r.min_key >> 4) << 4;
    const int64_t span = max<int64_t>(0, r.n_keys - r.key_begin);
    r.n_splits = max(1, static_cast<int>((span + a.split_keys - 1) / a.split_keys));
    return r;
}

constexpr int kMaxSplitKeys = 2048;
constexpr int kMaxSplitPages = kMaxSplitKeys / 16 + 2;

template <int D, int NB, int NT>
__global__ __launch_bounds__(256) void paged_decode_mfma_kernel(PagedArgs a) {
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    constexpr int kRow = 2 * D + 8;  // bytes per V row in LDS (8-byte pad: conflict-free transposed reads)
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform: scalar tile bookkeeping
    const int split = blockIdx.x, kh = blockIdx.y, b = blockIdx.z;
    const int G = a.group;

    const int g = lane & 15;
    const int j = lane >> 4;
    const int tiles_pw = a.split_keys >> 6;  // tiles per wave (<= 32)

    // Issue the position, this wave's block ids and Q together.  With no
    // sliding window the split starts at split * split_keys whatever the
    // position, so the block-id loads need not wait for it.
    const int64_t pos = load_index(a.pos, a.pos_dt, b);
    int32_t blkv = -1;  // lane i: block id of this wave's tile i
    auto load_ids = [&](int64_t sb) {
        const int64_t t = sb + 16 * wave + 64 * lane;
        const int64_t page = t >> a.log2_page;
        blkv = (lane < tiles_pw && page < a.max_blocks) ? a.table[b * a.table_stride + page] : -1;
    };
    if (a.window == 0) load_ids(static_cast<int64_t>(split) * a.split_keys);
    // Q^T as B operands: column g, d = 32 kk + 8 j .. + 7
    uint4 qv[D / 32];
    if (g < G) {
        const uint4* qp = reinterpret_cast<const uint4*>(a.q + b * a.q_sb + (kh * G + g) * a.q_sh + 8 * j);
#pragma unroll
        for (int kk = 0; kk < D / 32; kk++) qv[kk] = qp[kk * 4];
    } else {
#pragma unroll
        for (int kk = 0; kk < D / 32; kk++) qv[kk] = make_uint4(0, 0, 0, 0);
    }
    if (pos < 0 && threadIdx.x == 0 && split == 0 && kh == 0)
        atomicOr(a.errw, static_cast<uint32_t>(SANDY_DEVERR_ATTN_POS));
    const SplitRange sr = split_range(a, pos);
    const int n_splits = sr.n_splits;
    const int64_t min_key = sr.min_key;
    if (pos < 0 || split >= n_splits) {
        // empty split slot: mark it so the merge needs no position
        for (int gg = threadIdx.x; gg < G; gg += 256) {
            const int64_t slot = (static_cast<int64_t>(b) * a.hq + kh * G + gg) * a.max_splits + split;
            a.ws_ml[slot * 2] = -INFINITY;
            a.ws_ml[slot * 2 + 1] = 0.0f;
        }
        return;
    }
    const int64_t s_begin = sr.key_begin + static_cast<int64_t>(split) * a.split_keys;
    const int64_t s_end = min(sr.n_keys, s_begin + a.split_keys);
    if (a.window != 0) load_ids(s_begin);
    {
        const int64_t t = s_begin + 16 * wave + 64 * lane;
        const bool used = lane < tiles_pw && t < s_end;
        const bool ok = blkv >= 0 && blkv < a.num_pages;
        if (used && !ok) atomicOr(a.errw, static_cast<uint32_t>(SANDY_DEVERR_BLOCK));
        if (!ok) blkv = -1;
    }
    auto blk_of = [&](int it) -> int32_t { return __builtin_amdgcn_readlane(blkv, it); };

    float m = -INFINITY, l = 0.0f;
    f32x4_t acc[D / 16];
#pragma unroll
    for (int t = 0; t < D / 16; t++) acc[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    unsigned char* vl = smem + wave * NB * 16 * kRow;  // this wave's V tiles

    // A batch of NB 16-key tiles: S^T on MFMA, one online-softmax update for
    // the whole batch (one cross-lane max and sum), V^T through LDS, PV on MFMA.
    auto compute_batch = [&](const TileRegs<D> (&buf)[NB], int it0) {
        const int64_t tb = s_begin + 16 * wave + 64 * it0;
        bool live_n[NB];
#pragma unroll
        for (int n = 0; n < NB; n++) live_n[n] = tb + 64 * n < s_end && blk_of(it0 + n) >= 0;
        float sv[NB][4];
        float mx = -INFINITY;
#pragma unroll
        for (int n = 0; n < NB; n++) {
            const int64_t t0 = tb + 64 * n;
            const bool live = live_n[n];
            f32x4_t sc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kk = 0; kk < D / 32; kk++)
                sc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, buf[n].k[kk]),
                                                             __builtin_bit_cast(bf16x8_t, qv[kk]), sc, 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int64_t key = t0 + 4 * j + i;
                const bool valid = live && key < s_end && key >= min_key;
                sv[n][i] = valid ? sc[i] * a.scale_log2 : -INFINITY;
                mx = fmaxf(mx, sv[n][i]);
            }
        }
        mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        // branch-free update (keeps the load/wait schedule straight-line)
        const float m_new = fmaxf(m, mx);
        float p[NB][4];
        float rs = 0.0f;
#pragma unroll
        for (int n = 0; n < NB; n++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float e2 = exp2f(sv[n][i] - m_new);
                p[n][i] = sv[n][i] == -INFINITY ? 0.0f : bf16_to_f32(f32_to_bf16(e2));
                rs += p[n][i];
            }
        rs += __shfl_xor(rs, 16, 64);
        rs += __shfl_xor(rs, 32, 64);
        const float alpha = m == -INFINITY ? (m_new == -INFINITY ? 1.0f : 0.0f) : exp2f(m - m_new);
        l = l * alpha + rs;
        m = m_new;
#pragma unroll
        for (int t = 0; t < D / 16; t++) acc[t] *= alpha;

        // V tiles -> LDS (row = key; masked keys zeroed so they cannot inject NaN)
#pragma unroll
        for (int n = 0; n < NB; n++) {
            const int64_t t0 = tb + 64 * n;
            const bool live = live_n[n];
            const int64_t vkey = t0 + (lane & 15);
            const bool vvalid = live && vkey < s_end && vkey >= min_key;
            unsigned char* row = vl + (n * 16 + (lane & 15)) * kRow + 16 * j;
#pragma unroll
            for (int kk = 0; kk < D / 32; kk++) {
                uint4 v = vvalid ? buf[n].v[kk] : make_uint4(0, 0, 0, 0);
                uint2* dst = reinterpret_cast<uint2*>(row + 64 * kk);
                dst[0] = make_uint2(v.x, v.y);
                dst[1] = make_uint2(v.z, v.w);
            }
        }
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int n = 0; n < NB; n++) {
            const short4_t pb = pack_p(p[n]);
#pragma unroll
            for (int t = 0; t < D / 16; t++) {
                short4_t va;
                const unsigned char* col = vl + n * 16 * kRow + 2 * (16 * t + (lane & 15));
#pragma unroll
                for (int i = 0; i < 4; i++) va[i] = *reinterpret_cast<const short*>(col + (4 * j + i) * kRow);
                acc[t] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(va, pb, acc[t], 0, 0, 0);
            }
        }
        __builtin_amdgcn_wave_barrier();
    };

    // Ping-pong batches of NB tiles: the next batch's loads are in flight
    // while the current batch is computed.  Wave w owns tiles w, w+4, ...
    TileRegs<D> bufA[NB], bufB[NB];
    auto load_batch = [&](TileRegs<D> (&buf)[NB], int it0) {
#pragma unroll
        for (int n = 0; n < NB; n++) {
            // unconditional: a tile past the split reads block 0 (blk -1) and is masked later
            const int64_t t = s_begin + 16 * wave + 64 * (it0 + n);
            load_tile<D>(a, t, t < s_end ? blk_of(it0 + n) : -1, kh, lane, buf[n]);
        }
    };
    // NT tiles per wave, fully unrolled: every load is unconditional and every
    // compute predicated, so the wait counts stay exact and the next batch's
    // loads remain in flight while the current batch computes.
    static_assert(NT % NB == 0, "tiles per wave must be a multiple of the batch");
    load_batch(bufA, 0);
#pragma unroll
    for (int it = 0; it < NT; it += 2 * NB) {
        if (it + NB < NT) load_batch(bufB, it + NB);
        compute_batch(bufA, it);
        if (it + NB < NT) {
            if (it + 2 * NB < NT) load_batch(bufA, it + 2 * NB);
            compute_batch(bufB, it + NB);
        }
    }

    // ---- merge the 4 waves through LDS (reuses the V staging area)
    __syncthreads();
    float* red = reinterpret_cast<float*>(smem);   // [4][G][D]
    float* ml = red + 4 * G * D;                    // [4][G][2]
    if (g < G) {
#pragma unroll
        for (int t = 0; t < D / 16; t++)
#pragma unroll
            for (int i = 0; i < 4; i++) red[(wave * G + g) * D + 16 * t + 4 * j + i] = acc[t][i];
        if (j == 0) {
            ml[(wave * G + g) * 2] = m;
            ml[(wave * G + g) * 2 + 1] = l;
        }
    }
    __syncthreads();
    const int hq = a.hq;
    for (int idx = threadIdx.x; idx < G * D; idx += 256) {
        const int gg = idx / D, d = idx % D;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < 4; w++) M = fmaxf(M, ml[(w * G + gg) * 2]);
        float O = 0.0f, L = 0.0f;
        if (M != -INFINITY) {
#pragma unroll
            for (int w = 0; w < 4; w++) {
                const float mw = ml[(w * G + gg) * 2];
                if (mw == -INFINITY) continue;
                const float f = exp2f(mw - M);
                O += red[(w * G + gg) * D + d] * f;
                L += ml[(w * G + gg) * 2 + 1] * f;
            }
        }
        const int h = kh * G + gg;
        if (a.fused_merge && n_splits == 1) {
            a.out[b * a.o_sb + h * a.o_sh + d] = f32_to_bf16(L > 0.0f ? O / L : 0.0f);
            continue;
        }
        const int64_t slot = (static_cast<int64_t>(b) * hq + h) * a.max_splits + split;
        if (a.fused_merge) {  // agent-coherent stores: visible to every XCD once complete
            __hip_atomic_store(&a.ws_o[slot * D + d], O, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (d == 0) {
                __hip_atomic_store(&a.ws_ml[slot * 2], M, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_store(&a.ws_ml[slot * 2 + 1], L, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        } else {
            a.ws_o[slot * D + d] = O;
            if (d == 0) {
                a.ws_ml[slot * 2] = M;
                a.ws_ml[slot * 2 + 1] = L;
            }
        }
    }
    if (!a.fused_merge || n_splits == 1) return;

    // Fused merge: the partial stores above are agent-coherent; once they have
    // completed, the last workgroup of this (sequence, kv head) to arrive reads
    // every split's partial with agent-coherent loads and writes the output.
    __shared__ int is_last;
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0) {
        const uint32_t prev = __hip_atomic_fetch_add(&a.counters[b * a.hkv + kh], 1u, __ATOMIC_RELAXED,
                                                     __HIP_MEMORY_SCOPE_AGENT);
        is_last = prev == static_cast<uint32_t>(n_splits - 1);
    }
    __syncthreads();
    if (!is_last) return;
    for (int idx = threadIdx.x; idx < G * D; idx += 256) {
        const int gg = idx / D, d = idx % D;
        const int h = kh * G + gg;
        const int64_t base = (static_cast<int64_t>(b) * hq + h) * a.max_splits;
        float M = -INFINITY, L = 0.0f, O = 0.0f;
        for (int s0 = 0; s0 < n_splits; s0 += 8) {
            float ms[8], ls[8], os[8];
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const bool in = s0 + u < n_splits;
                const int64_t slot = base + (in ? s0 + u : 0);
                ms[u] = in ? __hip_atomic_load(&a.ws_ml[slot * 2], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : -INFINITY;
                ls[u] = __hip_atomic_load(&a.ws_ml[slot * 2 + 1], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                os[u] = __hip_atomic_load(&a.ws_o[slot * D + d], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
#pragma unroll
            for (int u = 0; u < 8; u++) {
                if (ms[u] == -INFINITY) continue;
                const float mn = fmaxf(M, ms[u]);
                const float fo = M == -INFINITY ? 0.0f : exp2f(M - mn);
                const float fs = exp2f(ms[u] - mn);
                L = L * fo + ls[u] * fs;
                O = O * fo + os[u] * fs;
                M = mn;
            }
        }
        a.out[b * a.o_sb + h * a.o_sh + d] = f32_to_bf16(L > 0.0f ? O / L : 0.0f);
    }
    if (threadIdx.x == 0)
        __hip_atomic_store(&a.counters[b * a.hkv + kh], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Combines the split partials of one (sequence, q head): log-sum-exp merge of
// (max, sum, O[D]) over all max_splits slots (empty slots carry max = -inf),
// every load issued at once -- one memory round trip, no position read.
template <int D>
__global__ __launch_bounds__(64) void paged_decode_merge_kernel(PagedArgs a) {
    const int h = blockIdx.x, b = blockIdx.y;
    constexpr int PER = D / 64;  // head dims per thread
    const int64_t base = (static_cast<int64_t>(b) * a.hq + h) * a.max_splits;
    float M = -INFINITY, L = 0.0f, O[PER];
#pragma unroll
    for (int i = 0; i < PER; i++) O[i] = 0.0f;
    for (int s0 = 0; s0 < a.max_splits; s0 += 8) {
        float ms[8], ls[8], os[8][PER];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const bool in = s0 + u < a.max_splits;
            const int64_t slot = base + (in ? s0 + u : 0);
            const float2 ml = *reinterpret_cast<const float2*>(a.ws_ml + slot * 2);
            ms[u] = in ? ml.x : -INFINITY;
            ls[u] = ml.y;
#pragma unroll
            for (int i = 0; i < PER; i++) os[u][i] = a.ws_o[slot * D + threadIdx.x + 64 * i];
        }
#pragma unroll
        for (int u = 0; u < 8; u++) {
            if (ms[u] == -INFINITY) continue;  // empty slot: its O was never written
            const float mn = fmaxf(M, ms[u]);
            const float fo = M == -INFINITY ? 0.0f : exp2f(M - mn);
            const float fs = exp2f(ms[u] - mn);
            L = L * fo + ls[u] * fs;
#pragma unroll
            for (int i = 0; i < PER; i++) O[i] = O[i] * fo + os[u][i] * fs;
            M = mn;
        }
    }
#pragma unroll
    for (int i = 0; i < PER; i++)
        a.out[b * a.o_sb + h * a.o_sh + threadIdx.x + 64 * i] = f32_to_bf16(L > 0.0f ? O[i] / L : 0.0f);
}

// ---------------------------------------------------------------- general kernel
struct GenArgs {
    const void* q;
    int64_t qs[4];  // strides over (b, h, qi, d)
    void* out;
    int64_t os[4];
    const void* k;
    const void* v;
    int64_t ks[4];  // dense strides over (b, kh, key, d)
    int64_t vs[4];
    int32_t dt;
    int32_t paged;
    // paged cache (decode only)
    int64_t page_elems;
    int64_t page_size;
    int64_t num_pages;
    const int32_t* table;
    int64_t table_stride;
    int64_t max_blocks;
    const void* pos;
    int32_t pos_dt;
    int32_t hq, hkv, tq;
    int64_t tk;  // dense key count (paged: max_blocks * page_size)
    int64_t d;
    int64_t window;
    float scale;
    float* scores;  // [B, Hq, Tq, tk]
    uint32_t* errw;
};

template <typename T>
__device__ __forceinline__ float kv_load(const GenArgs& a, const void* base, const int64_t* st, int b, int kh,
                                         int64_t key, int64_t d, bool& ok) {
    if (!a.paged) return Vec8<T>::load1(base, b * st[0] + kh * st[1] + key * st[2] + d * st[3]);
    const int64_t page = key / a.page_size;
    const int32_t blk = a.table[b * a.table_stride + page];
    if (blk < 0 || blk >= a.num_pages) {
        ok = false;
        return 0.0f;
    }
    return Vec8<T>::load1(base, static_cast<int64_t>(blk) * a.page_elems + (kh * a.page_size + key % a.page_size) * a.d + d);
}

template <typename T>
__global__ __launch_bounds__(256) void attention_general_kernel(GenArgs a) {
    __shared__ float fred[4];
    __shared__ double dred[4];
    const int qi = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const int tid = threadIdx.x;
    const int kh = h / (a.hq / a.hkv);
    int64_t base_pos = 0;
    if (a.pos) {
        base_pos = load_index(a.pos, a.pos_dt, b);
        if (base_pos < 0) {
            if (tid == 0) atomicOr(a.errw, static_cast<uint32_t>(SANDY_DEVERR_ATTN_POS));
            return;
        }
    }
    const int64_t qpos = base_pos + qi;
    const int64_t min_key = a.window > 0 ? max<int64_t>(0, qpos + 1 - a.window) : 0;
    const int64_t tk = a.tk;
    float* sc = a.scores + ((static_cast<int64_t>(b) * a.hq + h) * a.tq + qi) * tk;
    const int64_t qoff = b * a.qs[0] + h * a.qs[1] + qi * a.qs[2];
    float lmax = -INFINITY;
    bool ok = true;
    for (int64_t key = tid; key < tk; key += 256) {
        float s = -INFINITY;
        if (key <= qpos && key >= min_key) {
            float acc = 0.0f;
            for (int64_t d = 0; d < a.d; d++)
                acc = __fadd_rn(acc, __fmul_rn(Vec8<T>::load1(a.q, qoff + d * a.qs[3]),
                                               kv_load<T>(a, a.k, a.ks, b, kh, key, d, ok)));
            s = __fmul_rn(acc, a.scale);
        }
        sc[key] = s;
        lmax = fmaxf(lmax, s);
    }
    if (!ok) atomicOr(a.errw, static_cast<uint32_t>(SANDY_DEVERR_BLOCK));
    lmax = wave_max(lmax);
    if ((tid & 63) == 0) fred[tid >> 6] = lmax;
    __syncthreads();
    const float mx = fmaxf(fmaxf(fred[0], fred[1]), fmaxf(fred[2], fred[3]));
    const int64_t ooff = b * a.os[0] + h * a.os[1] + qi * a.os[2];
    if (mx == -INFINITY) {
        for (int64_t d = tid; d < a.d; d += 256) Vec8<T>::store1(a.out, ooff + d * a.os[3], 0.0f);
        return;
    }
    double sum = 0.0;
    for (int64_t key = tid; key < tk; key += 256) sum += exp(static_cast<double>(__fsub_rn(sc[key], mx)));
    sum = wave_sum(sum);
    if ((tid & 63) == 0) dred[tid >> 6] = sum;
    __syncthreads();
    const double total = dred[0] + dred[1] + dred[2] + dred[3];
    for (int64_t d = tid; d < a.d; d += 256) {
        float acc = 0.0f;
        if (total != 0.0) {
            const float inv = 1.0f / static_cast<float>(total);
            for (int64_t key = 0; key < tk; key++) {
                const float s = sc[key];
                if (s == -INFINITY) continue;
                const float prob = __fmul_rn(expf(__fsub_rn(s, mx)), inv);
                acc = __fadd_rn(acc, __fmul_rn(prob, kv_load<T>(a, a.v, a.vs, b, kh, key, d, ok)));
            }
        }
        Vec8<T>::store1(a.out, ooff + d * a.os[3], acc);
    }
}

int env_int(const char* name, int dflt) {
    const char* v = std::getenv(name);
    return v ? std::atoi(v) : dflt;
}

} // namespace
} // namespace sandy_hip

using namespace sandy_hip;

extern "C" int sandy_hip_attention(const SandyTensor* q, const SandyTensor* k, const SandyTensor* v,
                                   const SandyTensor* position_offsets, int64_t window, double scale,
                                   const SandyTensor* out, void* stream_, char* err, size_t err_cap) {
    Err e{err, err_cap};
    hipStream_t stream = static_cast<hipStream_t>(stream_);
    if (!valid_rank(q) || !valid_rank(k) || !valid_rank(v) || !valid_rank(out))
        return fail(e, SANDY_ERR_INVALID, "attention tensor rank out of range");
    if (!is_float(q->dtype) || !is_float(k->dtype) || !is_float(v->dtype))
        return fail(e, SANDY_ERR_INVALID, "attention q unsupported dtype");
    if (q->dtype != k->dtype || q->dtype != v->dtype) return fail(e, SANDY_ERR_INVALID, "attention operands must have same dtype");
    const int rank = q->rank;
    if ((rank != 3 && rank != 4) || k->rank != rank || v->rank != rank)
        return fail(e, SANDY_ERR_INVALID, "attention q, k, and v must all have rank 3 or rank 4");
    if (window < 0) return fail(e, SANDY_ERR_INVALID, "attention window must be >= 0");
    const int o = rank == 4 ? 1 : 0;
    const int64_t B = rank == 4 ? q->dims[0] : 1;
    if (rank == 4 && (k->dims[0] != B || v->dims[0] != B)) return fail(e, SANDY_ERR_INVALID, "attention batch dimension mismatch");
    const int64_t hq = q->dims[o], hkv = k->dims[o], tq = q->dims[o + 1], tk = k->dims[o + 1], D = q->dims[o + 2];
    if (v->dims[o] != hkv) return fail(e, SANDY_ERR_INVALID, "attention k and v head count mismatch");
    if (v->dims[o + 1] != tk) return fail(e, SANDY_ERR_INVALID, "attention k and v sequence dimension mismatch");
    if (k->dims[o + 2] != D || v->dims[o + 2] != D) return fail(e, SANDY_ERR_INVALID, "attention head dimension mismatch");
    if (hq <= 0 || hkv <= 0 || hq % hkv != 0) return fail(e, SANDY_ERR_INVALID, "attention heads must be divisible by kv_heads");
    if (!same_shape(*q, *out) || out->dtype != q->dtype) return fail(e, SANDY_ERR_INVALID, "attention output shape mismatch");
    if (position_offsets) {
        if (!is_index(position_offsets->dtype)) return fail(e, SANDY_ERR_INVALID, "attention position_offsets must be i32 or i64");
        const int64_t n = numel(*position_offsets);
        if (rank == 4 && n != B) return fail(e, SANDY_ERR_INVALID, "attention position_offsets length must match batch");
        if (rank == 3 && n != 1) return fail(e, SANDY_ERR_INVALID, "attention unbatched position_offsets must have one element");
        if (!contiguous(*position_offsets)) return fail(e, SANDY_ERR_UNSUPPORTED, "attention position_offsets must be contiguous");
    }
    if (numel(*q) == 0) return ok(e);
    int status = 0;
    uint32_t* errw = device_error_word(e, &status);
    if (status) return status;
    GenArgs a{};
    auto fill4 = [&](const SandyTensor* t, int64_t* s) {
        if (rank == 4) for (int i = 0; i < 4; i++) s[i] = t->strides[i];
        else { s[0] = 0; for (int i = 0; i < 3; i++) s[i + 1] = t->strides[i]; }
    };
    a.q = base_ptr(*q);
    fill4(q, a.qs);
    a.out = base_ptr(*out);
    fill4(out, a.os);
    a.k = base_ptr(*k);
    a.v = base_ptr(*v);
    fill4(k, a.ks);
    fill4(v, a.vs);
    a.dt = q->dtype;
    a.paged = 0;
    a.pos = position_offsets ? base_ptr(*position_offsets) : nullptr;
    a.pos_dt = position_offsets ? position_offsets->dtype : SANDY_I64;
    a.hq = static_cast<int32_t>(hq);
    a.hkv = static_cast<int32_t>(hkv);
    a.tq = static_cast<int32_t>(tq);
    a.tk = tk;
    a.d = D;
    a.window = window;
    a.scale = scale <= 0.0 ? 1.0f / sqrtf(static_cast<float>(D)) : static_cast<float>(scale);
    const size_t sbytes = static_cast<size_t>(B * hq * tq * std::max<int64_t>(tk, 1)) * sizeof(float);
    a.scores = static_cast<float*>(device_workspace(1, sbytes, stream, e, &status));
    if (status) return status;
    a.errw = errw;
    dim3 grid(static_cast<unsigned>(tq), static_cast<unsigned>(hq), static_cast<unsigned>(B));
    if (q->dtype == SANDY_BF16) hipLaunchKernelGGL(attention_general_kernel<BF16>, grid, dim3(256), 0, stream, a);
    else hipLaunchKernelGGL(attention_general_kernel<F32>, grid, dim3(256), 0, stream, a);
    SANDY_HIP_TRY(hipGetLastError(), e, "attention launch");
    return ok(e);
}

extern "C" int sandy_hip_paged_attention(const SandyTensor* q, const SandyPagedCache* kc, const SandyPagedCache* vc,
                                         const SandyTensor* table, const SandyTensor* position_offsets,
                                         int64_t window, double scale, const SandyTensor* out, void* stream_,
                                         char* err, size_t err_cap) {
    Err e{err, err_cap};
    hipStream_t stream = static_cast<hipStream_t>(stream_);
    if (!valid_rank(q) || !valid_rank(out) || !valid_rank(table) || !valid_rank(position_offsets) || !kc || !vc)
        return fail(e, SANDY_ERR_INVALID, "paged attention requires q, caches, block table, positions and output");
    if (!is_float(q->dtype)) return fail(e, SANDY_ERR_INVALID, "attention q unsupported dtype");
    if (kc->dtype != q->dtype || vc->dtype != q->dtype) return fail(e, SANDY_ERR_INVALID, "attention operands must have same dtype");
    if (q->rank != 4 || q->dims[2] != 1) return fail(e, SANDY_ERR_INVALID, "paged attention expects q [B, Hq, 1, D]");
    const int64_t B = q->dims[0], hq = q->dims[1], D = q->dims[3];
    const int64_t hkv = kc->prefix, P = kc->page_size;
    if (vc->prefix != hkv || vc->page_size != P || vc->inner != kc->inner || vc->num_pages != kc->num_pages)
        return fail(e, SANDY_ERR_INVALID, "attention k and v head count mismatch");
    if (kc->inner != D) return fail(e, SANDY_ERR_INVALID, "attention head dimension mismatch");
    if (P <= 0 || (P & (P - 1)) != 0) return fail(e, SANDY_ERR_INVALID, "paged tensor pool page_size must be a power of two");
    if (hq <= 0 || hkv <= 0 || hq % hkv != 0) return fail(e, SANDY_ERR_INVALID, "attention heads must be divisible by kv_heads");
    if (window < 0) return fail(e, SANDY_ERR_INVALID, "attention window must be >= 0");
    if (!same_shape(*q, *out) || out->dtype != q->dtype) return fail(e, SANDY_ERR_INVALID, "attention output shape mismatch");
    if (table->dtype != SANDY_I32 || table->rank != 2 || table->dims[0] != B || table->strides[1] != 1)
        return fail(e, SANDY_ERR_INVALID, "paged attention block table must be [B, max_blocks] int32 with unit inner stride");
    if (!is_index(position_offsets->dtype) || numel(*position_offsets) != B || !contiguous(*position_offsets))
        return fail(e, SANDY_ERR_INVALID, "attention position_offsets length must match batch");
    if (q->strides[3] != 1 || out->strides[3] != 1) return fail(e, SANDY_ERR_UNSUPPORTED, "paged attention needs unit head-dim stride");
    if (B == 0) return ok(e);
    int status = 0;
    uint32_t* errw = device_error_word(e, &status);
    if (status) return status;
    const int64_t G = hq / hkv;
    const int64_t max_blocks = table->dims[1];
    const float sc = scale <= 0.0 ? 1.0f / sqrtf(static_cast<float>(D)) : static_cast<float>(scale);

    const bool aligned = ((reinterpret_cast<uintptr_t>(base_ptr(*q)) | reinterpret_cast<uintptr_t>(kc->pool) |
                           reinterpret_cast<uintptr_t>(vc->pool)) & 15u) == 0 &&
                         q->strides[0] % 8 == 0 && q->strides[1] % 8 == 0;
    const bool mfma = q->dtype == SANDY_BF16 && (D == 64 || D == 128 || D == 256) && G <= 16 && P % 16 == 0 &&
                      aligned && env_int("SANDY_PAGED_GENERIC", 0) == 0;
    if (mfma) {
        PagedArgs a{};
        a.q = static_cast<const uint16_t*>(base_ptr(*q));
        a.q_sb = q->strides[0];
        a.q_sh = q->strides[1];
        a.out = static_cast<uint16_t*>(base_ptr(*out));
        a.o_sb = out->strides[0];
        a.o_sh = out->strides[1];
        a.k_pool = static_cast<const uint16_t*>(kc->pool);
        a.v_pool = static_cast<const uint16_t*>(vc->pool);
        a.page_elems = hkv * P * D;
        a.num_pages = kc->num_pages;
        a.table = static_cast<const int32_t*>(base_ptr(*table));
        a.table_stride = table->strides[0];
        a.max_blocks = max_blocks;
        a.pos = base_ptr(*position_offsets);
        a.pos_dt = position_offsets->dtype;
        a.page_size = static_cast<int32_t>(P);
        int lg = 0;
        while ((1LL << lg) < P) lg++;
        a.log2_page = lg;
        a.hq = static_cast<int32_t>(hq);
        a.hkv = static_cast<int32_t>(hkv);
        a.group = static_cast<int32_t>(G);
        a.window = window;
        a.scale_log2 = sc * kLog2e;
        // split size = 64 keys x tiles per wave (NT); ~4 workgroups per CU at the average context
        const int nb = D == 64 ? 2 : 1;
        const int64_t max_keys = max_blocks * P;
        int64_t split = env_int("SANDY_PAGED_SPLIT", 0);
        if (split <= 0) split = (max_keys * B * hkv) / 512;
        const int64_t nt = split <= 256 ? 4 : split <= 512 ? 8 : 16;
        split = 64 * nt;
        a.split_keys = static_cast<int32_t>(split);
        a.max_splits = static_cast<int32_t>((max_keys + split - 1) / split);
        const size_t ws_o = static_cast<size_t>(B * hq * a.max_splits * D) * sizeof(float);
        const size_t ws_ml = static_cast<size_t>(B * hq * a.max_splits * 2) * sizeof(float);
        char* ws = static_cast<char*>(device_workspace(0, ws_o + ws_ml, stream, e, &status));
        if (status) return status;
        a.ws_o = reinterpret_cast<float*>(ws);
        a.ws_ml = reinterpret_cast<float*>(ws + ws_o);
        a.errw = errw;
        a.fused_merge = env_int("SANDY_PAGED_FUSED_MERGE", 0);
        a.counters = static_cast<uint32_t*>(
            device_counters(0, static_cast<size_t>(B * hkv) * sizeof(uint32_t), stream, e, &status));
        if (status) return status;
        dim3 grid(static_cast<unsigned>(a.max_splits), static_cast<unsigned>(hkv), static_cast<unsigned>(B));
        const size_t lds_v = 4 * nb * 16 * (2 * D + 8);
        const size_t lds_r = (4 * G * D + 4 * G * 2) * sizeof(float);
        const size_t lds = std::max(lds_v, lds_r);
        dim3 mgrid(static_cast<unsigned>(hq), static_cast<unsigned>(B));
#define PD_LAUNCH(DD, NBB, NTT)                                                                          \
    hipLaunchKernelGGL((paged_decode_mfma_kernel<DD, NBB, NTT>), grid, dim3(256), lds, stream, a);        \
    if (!a.fused_merge) hipLaunchKernelGGL(paged_decode_merge_kernel<DD>, mgrid, dim3(64), 0, stream, a)
        if (D == 64) {
            if (nt == 4) { PD_LAUNCH(64, 2, 4); }
            else if (nt == 8) { PD_LAUNCH(64, 2, 8); }
            else { PD_LAUNCH(64, 2, 16); }
        } else if (D == 128) {
            if (nt == 4) { PD_LAUNCH(128, 1, 4); }
            else if (nt == 8) { PD_LAUNCH(128, 1, 8); }
            else { PD_LAUNCH(128, 1, 16); }
        } else {
            if (nt == 4) { PD_LAUNCH(256, 1, 4); }
            else if (nt == 8) { PD_LAUNCH(256, 1, 8); }
            else { PD_LAUNCH(256, 1, 16); }
        }
#undef PD_LAUNCH
        SANDY_HIP_TRY(hipGetLastError(), e, "paged attention launch");
        return ok(e);
    }
    GenArgs a{};
    a.q = base_ptr(*q);
    for (int i = 0; i < 4; i++) {
        a.qs[i] = q->strides[i];
        a.os[i] = out->strides[i];
    }
    a.out = base_ptr(*out);
    a.k = kc->pool;
    a.v = vc->pool;
    a.dt = q->dtype;
    a.paged = 1;
    a.page_elems = hkv * P * D;
    a.page_size = P;
    a.num_pages = kc->num_pages;
    a.table = static_cast<const int32_t*>(base_ptr(*table));
    a.table_stride = table->strides[0];
    a.max_blocks = max_blocks;
    a.pos = base_ptr(*position_offsets);
    a.pos_dt = position_offsets->dtype;
    a.hq = static_cast<int32_t>(hq);
    a.hkv = static_cast<int32_t>(hkv);
    a.tq = 1;
    a.tk = max_blocks * P;
    a.d = D;
    a.window = window;
    a.scale = sc;
    const size_t sbytes = static_cast<size_t>(B * hq * std::max<int64_t>(a.tk, 1)) * sizeof(float);
    a.scores = static_cast<float*>(device_workspace(1, sbytes, stream, e, &status));
    if (status) return status;
    a.errw = errw;
    dim3 grid(1, static_cast<unsigned>(hq), static_cast<unsigned>(B));
    if (q->dtype == SANDY_BF16) hipLaunchKernelGGL(attention_general_kernel<BF16>, grid, dim3(256), 0, stream, a);
    else hipLaunchKernelGGL(attention_general_kernel<F32>, grid, dim3(256), 0, stream, a);
    SANDY_HIP_TRY(hipGetLastError(), e, "paged attention launch");
    return ok(e);
}
