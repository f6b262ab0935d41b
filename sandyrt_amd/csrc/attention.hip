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
//   - K tiles of 16 keys are read from their page with 128-bit buffer loads
//     (a resource per tile; tiles past the unit get an empty range and
//     cost no memory traffic) straight into MFMA A operands; S^T = K Q^T on v_mfma_f32_16x16x32_bf16 (the head
//     group padded to 16 columns);
//   - online softmax in the exp2 domain, per q head (one MFMA column);
//   - P^T leaves the S^T MFMA already in the B-operand layout of
//     v_mfma_f32_16x16x16_bf16, and V tiles are transposed through LDS into A
//     operands with gfx950's transposing ds_read_b64_tr_b16 (one read per
//     16 x 4 operand), so O^T += V^T P^T runs on MFMA with no register
//     shuffles;
//   - work units (sequence, split, kv head) are numbered over the active
//     splits only, from a prefix scan of the positions, so workgroup ids --
//     dealt round-robin to the 8 XCDs -- spread the real work evenly across
//     XCDs and CUs whatever the context lengths; block ids and Q are then
//     fetched together, and each wave keeps a ring of batches of tiles in
//     flight while computing;
//   - the 4 waves merge in LDS; a sequence of one split is written as final
//     output, otherwise every unit writes a (max, sum, O[D]) partial to a
//     persistent workspace, written through to the agent's coherence point,
//     and the last of the sequence's workgroups for that kv head (an
//     arrival counter) merges the splits (log-sum-exp) and writes the rows
//     -- one launch.  The two-launch form (partials, then a merge kernel
//     reading the position alongside the first partials) is kept behind
//     SANDY_PAGED_FUSED_MERGE=0.  No host round trip and no allocation per
//     call.
// The probabilities enter the PV product as two bf16 operands (hi + lo), so
// P keeps about 17 bits and the normaliser is the float sum of the same p.
#include "common.h"

#include <algorithm>
#include <cstdlib>
#include <mutex>
#include <vector>

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
    int64_t page_elems;  // elements from one page to the next
    int64_t num_pages;
    const int32_t* table;
    int64_t table_stride;
    int64_t max_blocks;
    const void* pos;
    int32_t pos_dt;
    int32_t page_size;
    int32_t log2_page;
    int32_t hq, hkv, group;
    int32_t batch;
    int64_t window;
    float scale_log2;  // scale * log2(e)
    int32_t split_keys;  // split-unit schedule: keys per split
    int32_t max_splits;  // split-unit schedule: slots per (sequence, q head)
    // partial (O[D], max, sum) slots: [B, Hq, max_splits] for the split-unit
    // schedule, [workgroups, 2, G] for the balanced one
    float* ws_o;
    float* ws_ml;
    uint32_t* errw;
    uint32_t* counters;  // [B, Hkv] arrivals for the fused merge (zero between launches)
    int32_t fused;       // merge in the last-arriving workgroup of each (sequence, kv head)
    // The reference's own paged tensor (CudaPagedTensor.cpp:187-226, addressed as
    // CudaKernelUtils.cuh:82-108): when k_pages is set, page ordinal p of K
    // (of V) starts at k_pages[p] (v_pages[p]), one page list for the whole
    // batch, and sequence b's kv head kh is page row b * kv_rows_b + kh.
    // Otherwise pages are block ids into k_pool / v_pool, one table row per
    // sequence, and kv_rows_b is 0.
    const uint64_t* k_pages;
    const uint64_t* v_pages;
    int32_t kv_rows_b;
    int64_t tk;  // logical length of the grow dimension: keys at or past it never attend
};

// p = hi + lo with hi = bf16(p) and lo = bf16(p - hi): two bf16 MFMA operands
// that carry p to about 2^-17 relative, so P.V on bf16 MFMA keeps the float
// probabilities of the reference (TensorCalc.cpp:1167-1314) instead of
// bf16-rounded ones.
__device__ __forceinline__ void split_p(const float (&p)[4], short4_t& hi, short4_t& lo) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint16_t h = f32_to_bf16(p[i]);
        hi[i] = static_cast<short>(h);
        lo[i] = static_cast<short>(f32_to_bf16(p[i] - bf16_to_f32(h)));
    }
}

template <int D>
struct TileRegs {
    uint4 k[D / 32];
    uint4 v[D / 32];
};

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
constexpr int kBufferWord3 = 0x00020000;  // gfx9 buffer resource word 3: raw dword access

// Loads one 16-key tile of K and V of kv head kh from block `blk` (this
// lane: key lane%16, 8 dims per MFMA k-step) through buffer resources that
// span exactly the tile.  blk < 0 gives an empty range: the loads return
// zeros without touching memory, so tiles past a piece cost no bandwidth and
// every load can stay unconditional.
template <int D>
__device__ __forceinline__ void load_tile(const PagedArgs& a, uint64_t kpage, uint64_t vpage, int64_t in_page, int row,
                                          int lane, TileRegs<D>& r) {
    const int64_t off = (static_cast<int64_t>(row) * a.page_size + in_page) * D;
    const int bytes = kpage == 0 ? 0 : 32 * D;
    uint16_t* kp = kpage == 0 ? const_cast<uint16_t*>(a.q) : reinterpret_cast<uint16_t*>(kpage) + off;
    uint16_t* vp = kpage == 0 ? const_cast<uint16_t*>(a.q) : reinterpret_cast<uint16_t*>(vpage) + off;
    const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(kp, 0, bytes, kBufferWord3);
    const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(vp, 0, bytes, kBufferWord3);
    const int voff = ((lane & 15) * D + 8 * (lane >> 4)) * 2;
#pragma unroll
    for (int kk = 0; kk < D / 32; kk++) {
        r.k[kk] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rk, voff + 64 * kk, 0, 0));
        r.v[kk] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rv, voff + 64 * kk, 0, 0));
    }
}

// Keys of sequence b: [key_begin, n_keys) in 16-key tiles from key_begin
// (min_key is the first unmasked key under a sliding window).
struct SplitRange {
    int64_t n_keys, min_key, key_begin;
    int n_tiles;
};

__device__ __forceinline__ SplitRange seq_range(const PagedArgs& a, int64_t pos) {
    SplitRange r;
    r.n_keys = min(min(pos + 1, a.max_blocks * static_cast<int64_t>(a.page_size)), a.tk);
    r.min_key = a.window > 0 ? max<int64_t>(0, pos + 1 - a.window) : 0;
    r.key_begin = (r.min_key >> 4) << 4;
    const int64_t span = max<int64_t>(0, r.n_keys - r.key_begin);
    r.n_tiles = static_cast<int>((span + 15) >> 4);
    return r;
}

// Position of sequence i as a 64-bit value in this lane (i must be < batch).
// Plain loads: positions are read-only here and stay in L2.
__device__ __forceinline__ int64_t lane_position(const PagedArgs& a, int64_t i) {
    return a.pos_dt == SANDY_I32 ? static_cast<int64_t>(static_cast<const int32_t*>(a.pos)[i])
                                 : static_cast<const int64_t*>(a.pos)[i];
}

// Position i as two raw 32-bit words fetched with relaxed agent-scope atomic
// loads from branch-free addresses: they stay on the vector memory path, so
// a uniform position travels with the loads issued after it instead of
// being waited on (as a scalar load) before them.  join_position() combines
// them at the first use.
struct PosWords {
    uint32_t lo, hi;
};

__device__ __forceinline__ PosWords vector_position(const PagedArgs& a, int64_t i) {
    const bool i32 = a.pos_dt == SANDY_I32;
    uint32_t* p = reinterpret_cast<uint32_t*>(const_cast<void*>(a.pos)) + (i32 ? i : 2 * i);
    PosWords w;
    w.lo = __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    w.hi = __hip_atomic_load(p + (i32 ? 0 : 1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return w;
}

__device__ __forceinline__ int64_t join_position(const PagedArgs& a, PosWords w) {
    const uint32_t lo = __builtin_amdgcn_readfirstlane(w.lo);
    const uint32_t hi = a.pos_dt == SANDY_I32 ? static_cast<uint32_t>(static_cast<int32_t>(lo) >> 31)
                                              : __builtin_amdgcn_readfirstlane(w.hi);
    return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
}

__device__ __forceinline__ int64_t lane_read64(int64_t v, int l) {
    const uint32_t lo = __builtin_amdgcn_readlane(static_cast<uint32_t>(v), l);
    const uint32_t hi = __builtin_amdgcn_readlane(static_cast<uint32_t>(static_cast<uint64_t>(v) >> 32), l);
    return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
}

// One piece of work: tiles [tile_a, tile_b) of (sequence b, kv head kh) for
// the whole GQA group, at most 4 * NT tiles.  The 4 waves take tiles tile_a + wave + 4i; each keeps
// a ring of S batches of NB tiles in flight while it computes (S*NB*4 KB per
// wave at D = 64), with S^T = K Q^T and O^T += V^T P^T on MFMA and the online
// softmax in the exp2 domain.  The waves merge through LDS and the piece ends
// as the final output rows (final_out) or as partial slots slot0 + g*stride.
template <int D>
__device__ __forceinline__ void load_q_columns(const PagedArgs& a, int b, int kh, int lane, uint4 (&qv)[D / 32]) {
    // Q^T as B operands: column g, d = 32 kk + 8 j .. + 7.  Pad columns
    // (g >= G) load head 0 again: every column is independent through the
    // softmax and PV products, and pad columns are never stored.
    const int G = a.group, g = lane & 15, j = lane >> 4;
    const uint4* qp = reinterpret_cast<const uint4*>(a.q + b * a.q_sb + (kh * G + (g < G ? g : 0)) * a.q_sh + 8 * j);
#pragma unroll
    for (int kk = 0; kk < D / 32; kk++) qv[kk] = qp[kk * 4];
}

// Raw page-table word(s) of a tile's page: the K and V page addresses (the
// reference's paged tensor) or the block id (pool mode, low 32 bits of k).
struct PageRaw {
    uint64_t k, v;
};

__device__ __forceinline__ PageRaw load_page_raw(const PagedArgs& a, int b, int64_t page) {
    PageRaw r;
    if (a.k_pages) {
        r.k = a.k_pages[page];
        r.v = a.v_pages[page];
    } else {
        r.k = static_cast<uint32_t>(a.table[b * a.table_stride + page]);
        r.v = 0;
    }
    return r;
}

// PRE: the caller requested this lane's raw page words (pre) for tile
// tile_a + wave + 4 * lane, page (16 * tile) >> log2_page clamped below
// max_blocks, before the sequence's position was known (no sliding window:
// key_begin is 0); otherwise they are loaded here.
template <int D, int NB, int NT, int S, bool PRE = false>
__device__ __forceinline__ void attend_piece(const PagedArgs& a, unsigned char* smem, int lane, int wave, int b,
                                             int kh, const SplitRange& sr, int64_t tile_a, int64_t tile_b,
                                             bool final_out, int64_t slot0, int64_t slot_stride, bool coherent,
                                             PageRaw pre = PageRaw{0, 0}) {
    constexpr int kRow = 2 * D + 8;  // bytes per V row in LDS (8-byte pad: conflict-free transposed reads)
    const int G = a.group;
    const int g = lane & 15;
    const int j = lane >> 4;

    uint4 qv[D / 32];
    load_q_columns<D>(a, b, kh, lane, qv);

    float m = -INFINITY, l = 0.0f;
    f32x4_t acc[D / 16];
#pragma unroll
    for (int t = 0; t < D / 16; t++) acc[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    unsigned char* vl = smem + wave * NB * 16 * kRow;  // this wave's V tiles

    {
        const int64_t c0 = tile_a;  // tile_b - tile_a <= 4 * NT: one pass of the ring
        // lane i: start addresses of the K and V pages of this wave's tile i (0: none / invalid)
        uint64_t kpv, vpv;
        {
            const int64_t tile = c0 + wave + 4 * lane;
            const int64_t page = (sr.key_begin + 16 * tile) >> a.log2_page;
            // a tile wholly below a sliding window's first key needs no data
            const bool in = lane < NT && tile < tile_b && page < a.max_blocks &&
                            sr.key_begin + 16 * tile + 15 >= sr.min_key;
            bool ok;
            const PageRaw raw = PRE ? pre : load_page_raw(a, b, in ? page : 0);  // max_blocks >= 1
            if (a.k_pages) {
                kpv = raw.k;
                vpv = raw.v;
                // 16-byte buffer loads: a page that is null or not 16-byte aligned
                // is reported like a block id outside the pool
                ok = kpv != 0 && vpv != 0 && ((kpv | vpv) & 15u) == 0;
            } else {
                const int32_t id = static_cast<int32_t>(static_cast<uint32_t>(raw.k));
                ok = id >= 0 && id < a.num_pages;
                kpv = reinterpret_cast<uint64_t>(a.k_pool + static_cast<int64_t>(ok ? id : 0) * a.page_elems);
                vpv = reinterpret_cast<uint64_t>(a.v_pool + static_cast<int64_t>(ok ? id : 0) * a.page_elems);
            }
            if (in && !ok) atomicOr(a.errw, static_cast<uint32_t>(SANDY_DEVERR_BLOCK));
            if (!(in && ok)) kpv = vpv = 0;
        }
        const int row = b * a.kv_rows_b + kh;  // page row of (sequence b, kv head kh)
        auto kpage_of = [&](int it) -> uint64_t { return static_cast<uint64_t>(lane_read64(static_cast<int64_t>(kpv), it)); };
        auto vpage_of = [&](int it) -> uint64_t { return static_cast<uint64_t>(lane_read64(static_cast<int64_t>(vpv), it)); };
        auto blk_of = [&](int it) -> int32_t { return kpage_of(it) != 0 ? 0 : -1; };
        // key indices fit 32 bits (the host keeps max_blocks * page_size below 2^31)
        const int n_keys = static_cast<int>(sr.n_keys), min_key = static_cast<int>(sr.min_key);
        auto key0_of = [&](int it) -> int { return static_cast<int>(sr.key_begin + 16 * (c0 + wave + 4 * it)); };

        // A batch of NB tiles: S^T on MFMA, one online-softmax update for the
        // whole batch (one cross-lane max and sum), V^T through LDS, PV on MFMA.
        auto compute_batch = [&](const TileRegs<D> (&buf)[NB], int it0) {
            bool live_n[NB];
            bool any = false;
#pragma unroll
            for (int n = 0; n < NB; n++) {
                live_n[n] = blk_of(it0 + n) >= 0;
                any = any || live_n[n];
            }
            if (!any) return;  // wave-uniform
            float sv[NB][4];
            float mx = -INFINITY;
#pragma unroll
            for (int n = 0; n < NB; n++) {
                const int t0 = key0_of(it0 + n);
                f32x4_t sc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int kk = 0; kk < D / 32; kk++)
                    sc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, buf[n].k[kk]),
                                                                 __builtin_bit_cast(bf16x8_t, qv[kk]), sc, 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int key = t0 + 4 * j + i;
                    const bool valid = live_n[n] && key < n_keys && key >= min_key;
                    sv[n][i] = valid ? sc[i] * a.scale_log2 : -INFINITY;
                    mx = fmaxf(mx, sv[n][i]);
                }
            }
            mx = max_xor32(max_xor16(mx));
            const float m_new = fmaxf(m, mx);
            float p[NB][4];
            float rs = 0.0f;
#pragma unroll
            for (int n = 0; n < NB; n++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const float e2 = __builtin_amdgcn_exp2f(sv[n][i] - m_new);
                    p[n][i] = sv[n][i] == -INFINITY ? 0.0f : e2;
                    rs += p[n][i];
                }
            rs = sum_xor32(sum_xor16(rs));
            const float alpha = m == -INFINITY ? (m_new == -INFINITY ? 1.0f : 0.0f) : __builtin_amdgcn_exp2f(m - m_new);
            l = l * alpha + rs;
            m = m_new;
#pragma unroll
            for (int t = 0; t < D / 16; t++) acc[t] *= alpha;

            // V tiles -> LDS (row = key; masked keys zeroed so they cannot inject NaN)
#pragma unroll
            for (int n = 0; n < NB; n++) {
                const int vkey = key0_of(it0 + n) + (lane & 15);
                const bool vvalid = live_n[n] && vkey < n_keys && vkey >= min_key;
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
            // ds_read_b64_tr_b16: in each 16-lane group, lane i gets element i % 4 of the
            // 8-byte pieces addressed by lanes 4m + i / 4 (m = 0..3), so pointing lane i at
            // key 4j + i / 4, dims 16t + 4(i % 4) .. + 3 of tile n yields V[4j + m][16t + i], m = 0..3
            auto v_t = [&](int n, int t) -> short4_t {
                const int i = lane & 15;
                const unsigned char* src = vl + (n * 16 + 4 * j + (i >> 2)) * kRow + 2 * (16 * t + 4 * (i & 3));
                return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                    (short4_t __attribute__((address_space(3)))*)((unsigned char __attribute__((address_space(3)))*)src));
            };
            if constexpr (NB % 2 == 0) {
                // two tiles per v_mfma_f32_16x16x32_bf16 (twice the work of the 16x16x16 form in
                // the same passes on gfx950): contraction slot 8j + m holds key 4j + m of tile n
                // (m < 4) and of tile n + 1 (m >= 4), in V^T and P^T alike
#pragma unroll
                for (int n = 0; n < NB; n += 2) {
                    short4_t pb0, pl0, pb1, pl1;
                    split_p(p[n], pb0, pl0);
                    split_p(p[n + 1], pb1, pl1);
                    const bf16x8_t pb = __builtin_bit_cast(bf16x8_t, __builtin_shufflevector(pb0, pb1, 0, 1, 2, 3, 4, 5, 6, 7));
                    const bf16x8_t pl = __builtin_bit_cast(bf16x8_t, __builtin_shufflevector(pl0, pl1, 0, 1, 2, 3, 4, 5, 6, 7));
#pragma unroll
                    for (int t = 0; t < D / 16; t++) {
                        const bf16x8_t va =
                            __builtin_bit_cast(bf16x8_t, __builtin_shufflevector(v_t(n, t), v_t(n + 1, t), 0, 1, 2, 3, 4, 5, 6, 7));
                        acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, pb, acc[t], 0, 0, 0);
                        acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, pl, acc[t], 0, 0, 0);
                    }
                }
            } else {
#pragma unroll
                for (int n = 0; n < NB; n++) {
                    short4_t pb, pl;
                    split_p(p[n], pb, pl);
#pragma unroll
                    for (int t = 0; t < D / 16; t++) {
                        const short4_t va = v_t(n, t);
                        acc[t] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(va, pb, acc[t], 0, 0, 0);
                        acc[t] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(va, pl, acc[t], 0, 0, 0);
                    }
                }
            }
            __builtin_amdgcn_wave_barrier();
        };

        TileRegs<D> ring[S][NB];
        auto load_batch = [&](TileRegs<D> (&buf)[NB], int it0) {
#pragma unroll
            for (int n = 0; n < NB; n++)
                load_tile<D>(a, kpage_of(it0 + n), vpage_of(it0 + n), key0_of(it0 + n) & (a.page_size - 1), row, lane,
                             buf[n]);
        };
        // NT tiles per wave, fully unrolled: every load is unconditional (empty
        // ranges past the piece), so the wait counts stay exact and the later
        // batches' loads remain in flight while the current batch computes.
        static_assert(NT % NB == 0, "tiles per wave must be a multiple of the batch");
        constexpr int kBatches = NT / NB;
#pragma unroll
        for (int i = 0; i < S - 1; i++)
            if (i < kBatches) load_batch(ring[i], i * NB);
#pragma unroll
        for (int i = 0; i < kBatches; i++) {
            if (i + S - 1 < kBatches) load_batch(ring[(i + S - 1) % S], (i + S - 1) * NB);
            compute_batch(ring[i % S], i * NB);
        }
    }

    // ---- merge the 4 waves through LDS (reuses the V staging area)
    __syncthreads();
    float* red = reinterpret_cast<float*>(smem);  // [4][G][D]
    float* ml = red + 4 * G * D;                   // [4][G][2]
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
    for (int idx = threadIdx.x; idx < G * D / 2; idx += 256) {  // two dims per thread
        const int gg = idx / (D / 2), d = 2 * (idx % (D / 2));
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < 4; w++) M = fmaxf(M, ml[(w * G + gg) * 2]);
        float O0 = 0.0f, O1 = 0.0f, L = 0.0f;
        if (M != -INFINITY) {
#pragma unroll
            for (int w = 0; w < 4; w++) {
                const float mw = ml[(w * G + gg) * 2];
                if (mw == -INFINITY) continue;
                const float f = __builtin_amdgcn_exp2f(mw - M);
                O0 += red[(w * G + gg) * D + d] * f;
                O1 += red[(w * G + gg) * D + d + 1] * f;
                L += ml[(w * G + gg) * 2 + 1] * f;
            }
        }
        if (final_out) {
            const uint32_t pair = static_cast<uint32_t>(f32_to_bf16(L > 0.0f ? O0 / L : 0.0f)) |
                                  (static_cast<uint32_t>(f32_to_bf16(L > 0.0f ? O1 / L : 0.0f)) << 16);
            __builtin_nontemporal_store(pair, reinterpret_cast<uint32_t*>(&a.out[b * a.o_sb + (kh * G + gg) * a.o_sh + d]));
        } else {
            const int64_t slot = slot0 + gg * slot_stride;
            const uint64_t ov = static_cast<uint64_t>(__float_as_uint(O0)) | (static_cast<uint64_t>(__float_as_uint(O1)) << 32);
            const uint64_t mv = static_cast<uint64_t>(__float_as_uint(M)) | (static_cast<uint64_t>(__float_as_uint(L)) << 32);
            uint64_t* po = reinterpret_cast<uint64_t*>(&a.ws_o[slot * D + d]);
            uint64_t* pm = reinterpret_cast<uint64_t*>(&a.ws_ml[slot * 2]);
            if (coherent) {  // written through for a workgroup on another XCD (fused merge)
                __hip_atomic_store(po, ov, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                if (d == 0) __hip_atomic_store(pm, mv, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            } else {  // read by the merge kernel
                __builtin_nontemporal_store(ov, po);
                if (d == 0) __builtin_nontemporal_store(mv, pm);
            }
        }
    }
    __syncthreads();  // the next piece reuses the LDS
}

// Writes zeros for sequence b's rows (negative position) and raises the flag.
template <int D>
__device__ __forceinline__ void zero_rows(const PagedArgs& a, int b, int h) {
    for (int d = threadIdx.x; d < D; d += blockDim.x) a.out[b * a.o_sb + h * a.o_sh + d] = 0;
    if (h == 0 && threadIdx.x == 0) atomicOr(a.errw, static_cast<uint32_t>(SANDY_DEVERR_ATTN_POS));
}

// ------------------------------------------------ split-unit schedule (any B)
// Work units (sequence, split of 64*NT keys, kv head) are numbered over the
// active splits only (a prefix scan of the positions, 64 sequences at a
// time) and workgroup `lin` takes unit `lin`: consecutive workgroup ids are
// dealt round-robin to the 8 XCDs, so the active work spreads evenly over
// XCDs and CUs, and the idle workgroups are the last ones dispatched.
struct Unit {
    int b, kh, split;
    int64_t pos;
    bool active;
    int total;  // active units (set when !active)
};

// LPT: every sequence's whole splits first, then the shorter last splits, so
// the workgroups dispatched last carry the least work (the host picks it when
// the active units take more than one round of resident workgroups);
// otherwise each sequence's splits in order.
template <bool LPT>
__device__ __forceinline__ Unit find_unit(const PagedArgs& a, int lin, int split_tiles, int lane) {
    int base = 0;
#pragma unroll
    for (int phase = 0; phase < (LPT ? 2 : 1); phase++) {
        for (int c0 = 0; c0 < a.batch; c0 += 64) {
            const int bi = c0 + lane;
            const int64_t p = lane_position(a, bi < a.batch ? bi : 0);
            const bool live = bi < a.batch && p >= 0;
            const int n_tiles = live ? seq_range(a, p).n_tiles : 0;
            const int full = n_tiles / split_tiles;
            const int part = n_tiles % split_tiles != 0 ? 1 : 0;
            const int units = a.hkv * (!LPT ? full + part : phase == 0 ? full : part);
            int incl = units;
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const int t = __shfl_up(incl, o, 64);
                if (lane >= o) incl += t;
            }
            const int total = __builtin_amdgcn_readlane(incl, 63);
            if (lin < base + total) {
                const int bl = __builtin_ctzll(__ballot(lin < base + incl));
                const int r = lin - base - __builtin_amdgcn_readlane(incl - units, bl);
                Unit u;
                u.b = c0 + bl;
                u.split = phase == 0 ? r / a.hkv : __builtin_amdgcn_readlane(full, bl);
                u.kh = phase == 0 ? r - u.split * a.hkv : r;
                u.pos = lane_read64(p, bl);
                u.active = true;
                return u;
            }
            base += total;
        }
    }
    Unit u{};
    u.active = false;
    u.total = base;
    return u;
}

// The i-th sequence (in order) whose position is negative, or -1.  Such a
// sequence owns no work unit; under the fused merge an idle workgroup (there
// is at least one per such sequence) writes its zero rows and raises the
// error flag, which the merge kernel does otherwise.
__device__ __forceinline__ int negative_sequence(const PagedArgs& a, int i, int lane) {
    int base = 0;
    for (int c0 = 0; c0 < a.batch; c0 += 64) {
        const int bi = c0 + lane;
        const int64_t p = lane_position(a, bi < a.batch ? bi : 0);
        const uint64_t neg = __ballot(bi < a.batch && p < 0);
        const int cnt = __popcll(neg);
        if (i < base + cnt) {
            const int rank = __popcll(neg & ((1ull << lane) - 1));
            return c0 + __builtin_ctzll(__ballot(((neg >> lane) & 1) && rank == i - base));
        }
        base += cnt;
    }
    return -1;
}

// Fused split merge, run by every workgroup of a multi-split (sequence b,
// kv head kh) after it wrote its partial.  The partials were written through
// to the agent's coherence point; once every thread's stores have completed
// (the barrier waits for them), the workgroup counts itself in, and the last
// of the sequence's n_splits workgroups for this kv head reads every split's
// partial with agent-scope loads, writes the output rows and re-arms the
// counter for the next launch.
template <int D>
__device__ __forceinline__ void fused_merge(const PagedArgs& a, int b, int kh, int n_splits, int64_t slot0) {
    __shared__ int is_last;
    __builtin_amdgcn_s_waitcnt(0);  // this thread's write-through stores acknowledged
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t* ctr = a.counters + static_cast<int64_t>(b) * a.hkv + kh;
        const uint32_t prev = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        is_last = prev == static_cast<uint32_t>(n_splits - 1);
        if (is_last) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!is_last) return;
    const int G = a.group;
    for (int idx = threadIdx.x; idx < G * D / 2; idx += 256) {
        const int gg = idx / (D / 2), d = 2 * (idx % (D / 2));
        float M = -INFINITY, L = 0.0f, O0 = 0.0f, O1 = 0.0f;
        for (int s0 = 0; s0 < n_splits; s0 += 8) {
            uint64_t mv[8], ov[8];
#pragma unroll
            for (int q = 0; q < 8; q++) {
                const int64_t slot = slot0 + gg * a.max_splits + (s0 + q < n_splits ? s0 + q : 0);
                mv[q] = __hip_atomic_load(reinterpret_cast<uint64_t*>(&a.ws_ml[slot * 2]), __ATOMIC_RELAXED,
                                          __HIP_MEMORY_SCOPE_AGENT);
                ov[q] = __hip_atomic_load(reinterpret_cast<uint64_t*>(&a.ws_o[slot * D + d]), __ATOMIC_RELAXED,
                                          __HIP_MEMORY_SCOPE_AGENT);
            }
#pragma unroll
            for (int q = 0; q < 8; q++) {
                const float ms = __uint_as_float(static_cast<uint32_t>(mv[q]));
                if (s0 + q >= n_splits || ms == -INFINITY) continue;
                const float mn = fmaxf(M, ms);
                const float fo = M == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(M - mn);
                const float fs = __builtin_amdgcn_exp2f(ms - mn);
                L = L * fo + __uint_as_float(static_cast<uint32_t>(mv[q] >> 32)) * fs;
                O0 = O0 * fo + __uint_as_float(static_cast<uint32_t>(ov[q])) * fs;
                O1 = O1 * fo + __uint_as_float(static_cast<uint32_t>(ov[q] >> 32)) * fs;
                M = mn;
            }
        }
        const uint32_t pair = static_cast<uint32_t>(f32_to_bf16(L > 0.0f ? O0 / L : 0.0f)) |
                              (static_cast<uint32_t>(f32_to_bf16(L > 0.0f ? O1 / L : 0.0f)) << 16);
        *reinterpret_cast<uint32_t*>(&a.out[b * a.o_sb + (kh * G + gg) * a.o_sh + d]) = pair;
    }
}

// OCC: waves per SIMD the register allocation must allow (1 = no limit).  The
// D = 64 four-tile kernel (256-key splits) is held to 5, where it needs no
// scratch and 1280 of its workgroups are resident at once.
template <int D, int NB, int NT, int S, int OCC, bool LPT = false>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(OCC))) void paged_decode_units_kernel(PagedArgs a) {
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    constexpr int kSplitTiles = 4 * NT;  // the host passes split_keys == 16 * kSplitTiles
    const Unit u = find_unit<LPT>(a, blockIdx.x, kSplitTiles, lane);
    if (!u.active) {
        if (a.fused) {
            const int nb = negative_sequence(a, static_cast<int>(blockIdx.x) - u.total, lane);
            if (nb >= 0) {
                for (int idx = threadIdx.x; idx < a.hq * D; idx += 256) a.out[nb * a.o_sb + (idx / D) * a.o_sh + idx % D] = 0;
                if (threadIdx.x == 0) atomicOr(a.errw, static_cast<uint32_t>(SANDY_DEVERR_ATTN_POS));
            }
        }
        return;
    }
    const SplitRange sr = seq_range(a, u.pos);
    const int64_t ta = static_cast<int64_t>(u.split) * kSplitTiles;
    const int64_t tb = min<int64_t>(sr.n_tiles, ta + kSplitTiles);
    const int n_splits = (sr.n_tiles + kSplitTiles - 1) / kSplitTiles;
    const bool whole = n_splits == 1;
    const int64_t slot0 = (static_cast<int64_t>(u.b) * a.hq + u.kh * a.group) * a.max_splits;
    attend_piece<D, NB, NT, S>(a, smem, lane, wave, u.b, u.kh, sr, ta, tb, whole, slot0 + u.split, a.max_splits,
                               a.fused != 0);
    if (!a.fused || whole) return;
    fused_merge<D>(a, u.b, u.kh, n_splits, slot0);
}

// Static schedule for grids no larger than the CU count, with no sliding
// window: workgroup (sequence b, split, kv head) in sequence order over every
// split the block table can hold.  With no window a tile's page does not
// depend on the position, so each lane requests its tile's page-table word
// together with the position: the block ids arrive with it instead of one
// round trip later, and no scan of the positions precedes them.  A split past
// the sequence's length exits; under the fused merge, split 0 of a negative
// position writes its zero rows and raises the flag.  (On larger grids the
// idle splits interleaved with the active ones cost more than this saves.)
template <int D, int NB, int NT, int S, int OCC>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(OCC))) void paged_decode_static_kernel(PagedArgs a) {
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    constexpr int kSplitTiles = 4 * NT;  // the host passes split_keys == 16 * kSplitTiles
    const int lin = static_cast<int>(blockIdx.x);
    const int kh = lin % a.hkv;
    const int split = (lin / a.hkv) % a.max_splits;
    const int b = lin / (a.hkv * a.max_splits);
    const PosWords pw = vector_position(a, b);
    const int64_t ta = static_cast<int64_t>(split) * kSplitTiles;
    const int64_t page = min<int64_t>((16 * (ta + wave + 4 * lane)) >> a.log2_page, a.max_blocks - 1);
    const PageRaw raw = load_page_raw(a, b, page);
    const int64_t pos = join_position(a, pw);
    if (pos < 0) {
        if (a.fused && split == 0) {
            for (int idx = threadIdx.x; idx < a.group * D; idx += 256)
                a.out[b * a.o_sb + (kh * a.group + idx / D) * a.o_sh + idx % D] = 0;
            if (kh == 0 && threadIdx.x == 0) atomicOr(a.errw, static_cast<uint32_t>(SANDY_DEVERR_ATTN_POS));
        }
        return;
    }
    const SplitRange sr = seq_range(a, pos);
    const int n_splits = (sr.n_tiles + kSplitTiles - 1) / kSplitTiles;
    if (split >= n_splits) return;
    const int64_t tb = min<int64_t>(sr.n_tiles, ta + kSplitTiles);
    const bool whole = n_splits == 1;
    const int64_t slot0 = (static_cast<int64_t>(b) * a.hq + kh * a.group) * a.max_splits;
    attend_piece<D, NB, NT, S, true>(a, smem, lane, wave, b, kh, sr, ta, tb, whole, slot0 + split, a.max_splits,
                                     a.fused != 0, raw);
    if (!a.fused || whole) return;
    fused_merge<D>(a, b, kh, n_splits, slot0);
}

// Combines the split partials of one (sequence, q head) under the split-unit
// schedule.  The position is loaded with the first slots' partials (one
// memory round trip for up to 16 splits); slots at or past the sequence's
// split count hold stale data and are skipped by index, and a split whose
// keys were all masked carries max = -inf.  A sequence of one split was
// written as final output by its workgroup.
template <int D>
__global__ __launch_bounds__(64) void paged_decode_units_merge_kernel(PagedArgs a) {
    const int h = blockIdx.x, b = blockIdx.y;
    constexpr int PER = D / 64;  // head dims per thread
    const int64_t base = (static_cast<int64_t>(b) * a.hq + h) * a.max_splits;
    const PosWords pos_w = vector_position(a, b);
    const int split_tiles = a.split_keys >> 4;
    float M = -INFINITY, L = 0.0f, O[PER];
#pragma unroll
    for (int i = 0; i < PER; i++) O[i] = 0.0f;
    int64_t pos = -1;
    int n_splits = -1;  // known once the position has arrived (after the first loads)
    constexpr int R = 16;  // splits whose partials are loaded in one round trip
    for (int s0 = 0; s0 < a.max_splits; s0 += R) {
        float ms[R], ls[R], os[R][PER];
#pragma unroll
        for (int u = 0; u < R; u++) {
            const int64_t slot = base + (s0 + u < a.max_splits ? s0 + u : 0);
            const float2 v = *reinterpret_cast<const float2*>(a.ws_ml + slot * 2);
            ms[u] = v.x;
            ls[u] = v.y;
#pragma unroll
            for (int i = 0; i < PER; i++) os[u][i] = a.ws_o[slot * D + threadIdx.x + 64 * i];
        }
        if (n_splits < 0) {
            pos = join_position(a, pos_w);
            n_splits = pos < 0 ? 0 : (seq_range(a, pos).n_tiles + split_tiles - 1) / split_tiles;
        }
#pragma unroll
        for (int u = 0; u < R; u++) {
            if (s0 + u >= n_splits || ms[u] == -INFINITY) continue;
            const float mn = fmaxf(M, ms[u]);
            const float fo = M == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(M - mn);
            const float fs = __builtin_amdgcn_exp2f(ms[u] - mn);
            L = L * fo + ls[u] * fs;
#pragma unroll
            for (int i = 0; i < PER; i++) O[i] = O[i] * fo + os[u][i] * fs;
            M = mn;
        }
        if (s0 + R >= n_splits) break;
    }
    if (n_splits == 1) return;  // written as final output by its workgroup
    if (pos < 0 && h == 0 && threadIdx.x == 0) atomicOr(a.errw, static_cast<uint32_t>(SANDY_DEVERR_ATTN_POS));
    // (a negative position has no splits: L = 0 writes zeros)
#pragma unroll
    for (int i = 0; i < PER; i++)
        a.out[b * a.o_sb + h * a.o_sh + threadIdx.x + 64 * i] = f32_to_bf16(L > 0.0f ? O[i] / L : 0.0f);
}

// ------------------------------------------------ kernel selection (host)
template <int D, int NB, bool LPT>
const void* units_for(int nt) {
    constexpr int kOcc4 = D == 64 ? 5 : 1;  // spill-free only for D = 64, four tiles per wave
    if constexpr (D == 256) {
        // held to 2 waves per SIMD: 248 VGPRs and no spills, where the unbounded
        // allocation (246 VGPRs + 64 AGPRs) leaves one wave per SIMD -- twice the
        // resident units (config 4: 132.0 -> 122.9 us with 512-key splits)
        return nt == 2   ? reinterpret_cast<const void*>(&paged_decode_units_kernel<D, NB, 2, 2, 2, LPT>)
               : nt == 4 ? reinterpret_cast<const void*>(&paged_decode_units_kernel<D, NB, 4, 2, 2, LPT>)
               : nt == 8 ? reinterpret_cast<const void*>(&paged_decode_units_kernel<D, NB, 8, 2, 2, LPT>)
                         : reinterpret_cast<const void*>(&paged_decode_units_kernel<D, NB, 16, 2, 2, LPT>);
    }
    return nt == 2   ? reinterpret_cast<const void*>(&paged_decode_units_kernel<D, NB, 2, 2, kOcc4, LPT>)
           : nt == 4 ? reinterpret_cast<const void*>(&paged_decode_units_kernel<D, NB, 4, 2, kOcc4, LPT>)
           : nt == 8 ? reinterpret_cast<const void*>(&paged_decode_units_kernel<D, NB, 8, 2, 1, LPT>)
                     : reinterpret_cast<const void*>(&paged_decode_units_kernel<D, NB, 16, 2, 1, LPT>);
}

// the static-schedule kernels (same register bounds as units_for)
template <int D, int NB>
const void* static_for(int nt) {
    constexpr int kOcc4 = D == 64 ? 5 : 1;
    if constexpr (D == 256) {
        return nt == 2   ? reinterpret_cast<const void*>(&paged_decode_static_kernel<D, NB, 2, 2, 2>)
               : nt == 4 ? reinterpret_cast<const void*>(&paged_decode_static_kernel<D, NB, 4, 2, 2>)
               : nt == 8 ? reinterpret_cast<const void*>(&paged_decode_static_kernel<D, NB, 8, 2, 2>)
                         : reinterpret_cast<const void*>(&paged_decode_static_kernel<D, NB, 16, 2, 2>);
    }
    return nt == 2   ? reinterpret_cast<const void*>(&paged_decode_static_kernel<D, NB, 2, 2, kOcc4>)
           : nt == 4 ? reinterpret_cast<const void*>(&paged_decode_static_kernel<D, NB, 4, 2, kOcc4>)
           : nt == 8 ? reinterpret_cast<const void*>(&paged_decode_static_kernel<D, NB, 8, 2, 1>)
                     : reinterpret_cast<const void*>(&paged_decode_static_kernel<D, NB, 16, 2, 1>);
}

const void* static_kernel(int D, int nt) {
    return D == 64 ? static_for<64, 2>(nt) : D == 128 ? static_for<128, 1>(nt) : static_for<256, 1>(nt);
}

const void* units_kernel(int D, int nt, bool lpt = false) {
    if (lpt) return D == 64 ? units_for<64, 2, true>(nt) : D == 128 ? units_for<128, 1, true>(nt) : units_for<256, 1, true>(nt);
    return D == 64 ? units_for<64, 2, false>(nt) : D == 128 ? units_for<128, 1, false>(nt) : units_for<256, 1, false>(nt);
}

// CUs of the current device (256 on MI355X), read once.
int64_t device_cu_count() {
    static const int64_t cus = [] {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
            n = 256;
        return static_cast<int64_t>(n);
    }();
    return cus;
}

// Workgroups of 256 threads of kernel fn with `lds` bytes of dynamic LDS
// resident on the whole device at once (occupancy times CUs), cached.
int64_t resident_workgroups(const void* fn, size_t lds) {
    static std::mutex mu;
    static std::vector<std::pair<std::pair<const void*, size_t>, int64_t>> cache;
    std::lock_guard<std::mutex> lock(mu);
    for (const auto& c : cache)
        if (c.first.first == fn && c.first.second == lds) return c.second;
    int blocks = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, fn, 256, lds) != hipSuccess || blocks <= 0) blocks = 1;
    const int64_t n = static_cast<int64_t>(blocks) * device_cu_count();
    cache.push_back({{fn, lds}, n});
    return n;
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
    // the reference's paged tensor: page p of K (V) at k_pages[p] (v_pages[p]),
    // one page list for the batch, (b, kh) on page row b * kv_rows_b + kh;
    // k and v are then null and offsets are absolute element addresses
    const uint64_t* k_pages;
    const uint64_t* v_pages;
    int64_t kv_rows_b;
};

// Element offset of row (b, kh, key) of K or V and its head-dim stride;
// a paged key whose block id is outside the pool (or whose page address is
// null) clears `ok` (offset 0).
__device__ __forceinline__ int64_t kv_row(const GenArgs& a, const int64_t* st, const uint64_t* pages, int b, int kh,
                                          int64_t key, bool& ok) {
    if (!a.paged) return b * st[0] + kh * st[1] + key * st[2];
    // page_size is a power of two (checked on the host): shifts, not 64-bit divisions
    const int sh = __builtin_ctzll(static_cast<uint64_t>(a.page_size));
    const int64_t page = key >> sh, in_page = key & (a.page_size - 1);
    if (pages) {
        const uint64_t at = pages[page];
        if (at == 0) {
            // no page: flagged, and the row offset points at q (readable memory:
            // offsets are absolute element addresses here, and loads through
            // this row stay inside q's first row)
            ok = false;
            return static_cast<int64_t>(reinterpret_cast<uintptr_t>(a.q) >> (a.dt == SANDY_F32 ? 2 : 1));
        }
        return static_cast<int64_t>(at >> (a.dt == SANDY_F32 ? 2 : 1)) + ((b * a.kv_rows_b + kh) * a.page_size + in_page) * a.d;
    }
    const int32_t blk = a.table[b * a.table_stride + page];
    if (blk < 0 || blk >= a.num_pages) {
        ok = false;
        return 0;
    }
    return static_cast<int64_t>(blk) * a.page_elems + (kh * a.page_size + in_page) * a.d;
}

// The reference's algorithm per (query, head, batch), in its operation order:
// float scores q.k summed over d in order, times scale; masked keys -inf; max;
// a double sum of exp(s - max); out[d] = sum over unmasked keys in order of
// (expf(s - max) * (1 / (float)sum)) * v[key][d].  The order is kept, the
// latency is not: q sits in LDS, each key's row address is computed once,
// and K / V values are loaded 16 at a time ahead of the in-order sums (a
// masked key adds an exact +0.0 through a select instead of a branch).
template <typename T>
__global__ __launch_bounds__(256) void attention_general_kernel(GenArgs a) {
    constexpr int kU = 16;
    __shared__ float fred[4];
    __shared__ double dred[4];
    __shared__ float qv[512];
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
    const int64_t D = a.d;
    float* sc = a.scores + ((static_cast<int64_t>(b) * a.hq + h) * a.tq + qi) * tk;
    const int64_t qoff = b * a.qs[0] + h * a.qs[1] + qi * a.qs[2];
    for (int64_t d = tid; d < D; d += 256) qv[d] = Vec8<T>::load1(a.q, qoff + d * a.qs[3]);
    __syncthreads();
    const int64_t kd = a.paged ? 1 : a.ks[3];
    const int64_t vd = a.paged ? 1 : a.vs[3];
    float lmax = -INFINITY;
    bool ok = true;
    for (int64_t key = tid; key < tk; key += 256) {
        float s = -INFINITY;
        if (key <= qpos && key >= min_key) {
            const int64_t row = kv_row(a, a.ks, a.k_pages, b, kh, key, ok);
            float acc = 0.0f;
            int64_t d = 0;
            for (; d + kU <= D; d += kU) {
                float kv[kU];
#pragma unroll
                for (int j = 0; j < kU; j++) kv[j] = Vec8<T>::load1(a.k, row + (d + j) * kd);
#pragma unroll
                for (int j = 0; j < kU; j++) acc = __fadd_rn(acc, __fmul_rn(qv[d + j], kv[j]));
            }
            for (; d < D; d++) acc = __fadd_rn(acc, __fmul_rn(qv[d], Vec8<T>::load1(a.k, row + d * kd)));
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
        for (int64_t d = tid; d < D; d += 256) Vec8<T>::store1(a.out, ooff + d * a.os[3], 0.0f);
        return;
    }
    double sum = 0.0;
    for (int64_t key = tid; key < tk; key += 256) sum += exp(static_cast<double>(__fsub_rn(sc[key], mx)));
    sum = wave_sum(sum);
    if ((tid & 63) == 0) dred[tid >> 6] = sum;
    __syncthreads();
    const double total = dred[0] + dred[1] + dred[2] + dred[3];
    const float inv = total != 0.0 ? 1.0f / static_cast<float>(total) : 0.0f;
    // keys past the query's position or below the window are masked for every d
    const int64_t k_end = min<int64_t>(tk, qpos + 1);
    for (int64_t d = tid; d < D; d += 256) {
        float acc = 0.0f;
        if (total != 0.0) {
            for (int64_t k0 = min_key; k0 < k_end; k0 += kU) {
                float vv[kU], sv[kU];
#pragma unroll
                for (int j = 0; j < kU; j++) {
                    const int64_t key = k0 + j;
                    sv[j] = key < k_end ? sc[key] : -INFINITY;
                    vv[j] = 0.0f;
                    if (sv[j] != -INFINITY) vv[j] = Vec8<T>::load1(a.v, kv_row(a, a.vs, a.v_pages, b, kh, key, ok) + d * vd);
                }
#pragma unroll
                for (int j = 0; j < kU; j++) {
                    const float prob = __fmul_rn(expf(__fsub_rn(sv[j], mx)), inv);
                    acc = __fadd_rn(acc, sv[j] == -INFINITY ? 0.0f : __fmul_rn(prob, vv[j]));
                }
            }
        }
        Vec8<T>::store1(a.out, ooff + d * a.os[3], acc);
    }
    // V rows are looked up only here: a missing V page is flagged after the loop
    if (!ok) atomicOr(a.errw, static_cast<uint32_t>(SANDY_DEVERR_BLOCK));
}

// The same algorithm and operation order for up to kGenStage keys, with the
// round trips cut: each key's thread looks up its K and V rows once (paged:
// one block-table read each, issued together) and keeps the V row offset in
// LDS; the K row is requested 64 values at a time ahead of the in-order dot
// product; scores and probabilities stay in LDS; P.V reads 32 keys' values
// per batch, all in flight, from the staged offsets (clamped key, kept by a
// select).  Results are identical to attention_general_kernel.
constexpr int kGenStage = 2048;

template <typename T>
__global__ __launch_bounds__(256) void attention_staged_kernel(GenArgs a) {
    constexpr int kC = 64;  // K values in flight per key
    constexpr int kV = 32;  // keys per P.V batch
    __shared__ float fred[4];
    __shared__ double dred[4];
    __shared__ float qv[512];
    __shared__ float ssc[kGenStage];
    __shared__ float sprob[kGenStage];
    __shared__ int64_t svrow[kGenStage];
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
    const int64_t D = a.d;
    const int64_t qoff = b * a.qs[0] + h * a.qs[1] + qi * a.qs[2];
    for (int64_t d = tid; d < D; d += 256) qv[d] = Vec8<T>::load1(a.q, qoff + d * a.qs[3]);
    __syncthreads();
    const int64_t kd = a.paged ? 1 : a.ks[3];
    const int64_t vd = a.paged ? 1 : a.vs[3];
    float lmax = -INFINITY;
    bool ok = true;
    for (int64_t key = tid; key < tk; key += 256) {
        float s = -INFINITY;
        const bool live = key <= qpos && key >= min_key;
        const int64_t krow = live ? kv_row(a, a.ks, a.k_pages, b, kh, key, ok) : 0;
        svrow[key] = live ? kv_row(a, a.vs, a.v_pages, b, kh, key, ok) : 0;
        if (live) {
            float acc = 0.0f;
            for (int64_t d0 = 0; d0 < D; d0 += kC) {
                float kv[kC];
#pragma unroll
                for (int j = 0; j < kC; j++) kv[j] = Vec8<T>::load1(a.k, krow + (d0 + j < D ? d0 + j : D - 1) * kd);
#pragma unroll
                for (int j = 0; j < kC; j++)
                    if (d0 + j < D) acc = __fadd_rn(acc, __fmul_rn(qv[d0 + j], kv[j]));
            }
            s = __fmul_rn(acc, a.scale);
        }
        ssc[key] = s;
        lmax = fmaxf(lmax, s);
    }
    if (!ok) atomicOr(a.errw, static_cast<uint32_t>(SANDY_DEVERR_BLOCK));
    lmax = wave_max(lmax);
    if ((tid & 63) == 0) fred[tid >> 6] = lmax;
    __syncthreads();
    const float mx = fmaxf(fmaxf(fred[0], fred[1]), fmaxf(fred[2], fred[3]));
    const int64_t ooff = b * a.os[0] + h * a.os[1] + qi * a.os[2];
    if (mx == -INFINITY) {
        for (int64_t d = tid; d < D; d += 256) Vec8<T>::store1(a.out, ooff + d * a.os[3], 0.0f);
        return;
    }
    double sum = 0.0;
    for (int64_t key = tid; key < tk; key += 256) sum += exp(static_cast<double>(__fsub_rn(ssc[key], mx)));
    sum = wave_sum(sum);
    if ((tid & 63) == 0) dred[tid >> 6] = sum;
    __syncthreads();
    const double total = dred[0] + dred[1] + dred[2] + dred[3];
    const float inv = total != 0.0 ? 1.0f / static_cast<float>(total) : 0.0f;
    for (int64_t key = tid; key < tk; key += 256) sprob[key] = __fmul_rn(expf(__fsub_rn(ssc[key], mx)), inv);
    __syncthreads();
    const int64_t k_end = min<int64_t>(tk, qpos + 1);
    for (int64_t d = tid; d < D; d += 256) {
        float acc = 0.0f;
        if (total != 0.0) {
            for (int64_t k0 = min_key; k0 < k_end; k0 += kV) {
                float vv[kV];
#pragma unroll
                for (int j = 0; j < kV; j++) {
                    const int64_t key = k0 + j < k_end ? k0 + j : k_end - 1;
                    vv[j] = Vec8<T>::load1(a.v, svrow[key] + d * vd);
                }
#pragma unroll
                for (int j = 0; j < kV; j++) {
                    const int64_t key = k0 + j;
                    if (key >= k_end) break;
                    const float sv = ssc[key];
                    acc = __fadd_rn(acc, sv == -INFINITY ? 0.0f : __fmul_rn(sprob[key], vv[j]));
                }
            }
        }
        Vec8<T>::store1(a.out, ooff + d * a.os[3], acc);
    }
}

// fp32 single-query steps (decode, Tq = 1) with up to kGenStage keys, head
// dim 32 / 64 / 128 / 256: the GPT-2 decode attention.  The scores are the
// reference's -- one thread per key sums q.k over d in order (float, no
// contraction: bit for bit the reference's score) from 16-byte loads of its
// K row, all in flight -- and so are the max and the double sum of exp(s -
// max).  P.V spreads over every thread: 256 / D groups of D threads take
// consecutive key ranges, each summing its range in key order with all of
// its V rows requested at once, and the groups' partials are added in group
// order.  That last split is the only change of order against the
// reference's single in-order sum (fp32 rounding, not bit for bit).
template <int D>
__global__ __launch_bounds__(256) void attention_decode_f32_kernel(GenArgs a) {
    constexpr int kG = 256 / D;   // key groups in P.V
    constexpr int kB = 16;        // V rows per group in flight
    __shared__ float fred[4];
    __shared__ double dred[4];
    __shared__ __attribute__((aligned(16))) float qv[D];
    __shared__ float sprob[kGenStage];
    __shared__ int64_t svrow[kGenStage];
    __shared__ float part[kG][D];
    const int h = blockIdx.y, b = blockIdx.z;
    const int tid = threadIdx.x;
    const int kh = h / (a.hq / a.hkv);
    // requested together before any is waited for: the position's words
    // (relaxed atomic loads stay on the vector memory path), this thread's q
    // value and the block id of key tid's page -- with no window the first
    // keys are 0..255 whatever the position (clamped to the table's width)
    uint32_t plo = 0, phi = 0;
    if (a.pos) {
        const bool i32 = a.pos_dt == SANDY_I32;
        uint32_t* pp = reinterpret_cast<uint32_t*>(const_cast<void*>(a.pos)) + (i32 ? b : 2 * b);
        plo = __hip_atomic_load(pp, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        phi = __hip_atomic_load(pp + (i32 ? 0 : 1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    const float* qg = static_cast<const float*>(a.q) + b * a.qs[0] + h * a.qs[1];
    const float qt = qg[tid < D ? tid : 0];
    const int sh = __builtin_ctzll(static_cast<uint64_t>(a.page_size));  // a power of two (host-checked)
    const int32_t blk0 = a.max_blocks > 0 ? a.table[b * a.table_stride + min<int64_t>(tid >> sh, a.max_blocks - 1)] : -1;
    int64_t qpos = 0;
    if (a.pos) {
        qpos = a.pos_dt == SANDY_I32 ? static_cast<int64_t>(static_cast<int32_t>(plo))
                                     : static_cast<int64_t>((static_cast<uint64_t>(phi) << 32) | plo);
        if (qpos < 0) {
            if (tid == 0) atomicOr(a.errw, static_cast<uint32_t>(SANDY_DEVERR_ATTN_POS));
            return;
        }
    }
    const int64_t min_key = a.window > 0 ? max<int64_t>(0, qpos + 1 - a.window) : 0;
    const int64_t k_end = min<int64_t>(a.tk, qpos + 1);
    if (tid < D) qv[tid] = qt;
    __syncthreads();
    const float* kp = static_cast<const float*>(a.k);  // pool mode: k and v are the pools
    const float* vp = static_cast<const float*>(a.v);
    float lmax = -INFINITY;
    bool ok = true;
    for (int64_t key = min_key + tid; key < k_end; key += 256) {
        // pool mode: a key's K and V rows sit at the same offset of their pools
        int64_t krow;
        if (min_key == 0 && key == tid) {  // the block id requested up front
            const int64_t in_page = key & (a.page_size - 1);
            const bool bok = blk0 >= 0 && blk0 < a.num_pages;
            ok = ok && bok;
            krow = bok ? static_cast<int64_t>(blk0) * a.page_elems + (kh * a.page_size + in_page) * a.d : 0;
        } else {
            krow = kv_row(a, a.ks, a.k_pages, b, kh, key, ok);
        }
        svrow[key - min_key] = krow;
        const float4* kr = reinterpret_cast<const float4*>(kp + krow);
        float4 kv[D / 4];
#pragma unroll
        for (int j = 0; j < D / 4; j++) kv[j] = kr[j];
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < D / 4; j++) {
            acc = __fadd_rn(acc, __fmul_rn(qv[4 * j], kv[j].x));
            acc = __fadd_rn(acc, __fmul_rn(qv[4 * j + 1], kv[j].y));
            acc = __fadd_rn(acc, __fmul_rn(qv[4 * j + 2], kv[j].z));
            acc = __fadd_rn(acc, __fmul_rn(qv[4 * j + 3], kv[j].w));
        }
        const float sc = __fmul_rn(acc, a.scale);
        sprob[key - min_key] = sc;
        lmax = fmaxf(lmax, sc);
    }
    if (!ok) atomicOr(a.errw, static_cast<uint32_t>(SANDY_DEVERR_BLOCK));
    lmax = wave_max(lmax);
    if ((tid & 63) == 0) fred[tid >> 6] = lmax;
    __syncthreads();
    const float mx = fmaxf(fmaxf(fred[0], fred[1]), fmaxf(fred[2], fred[3]));
    float* og = static_cast<float*>(a.out) + b * a.os[0] + h * a.os[1];
    const int64_t n = max<int64_t>(0, k_end - min_key);
    if (mx == -INFINITY) {
        if (tid < D) og[tid] = 0.0f;
        return;
    }
    double sum = 0.0;
    for (int64_t i = tid; i < n; i += 256) sum += exp(static_cast<double>(__fsub_rn(sprob[i], mx)));
    sum = wave_sum(sum);
    if ((tid & 63) == 0) dred[tid >> 6] = sum;
    __syncthreads();
    const double total = dred[0] + dred[1] + dred[2] + dred[3];
    const float inv = 1.0f / static_cast<float>(total);
    for (int64_t i = tid; i < n; i += 256) sprob[i] = __fmul_rn(expf(__fsub_rn(sprob[i], mx)), inv);
    __syncthreads();
    // P.V: group g sums keys [g * per, (g + 1) * per) in order
    const int g = tid / D, d = tid % D;
    const int64_t per = (n + kG - 1) / kG;
    const int64_t i0 = g * per, i1 = min<int64_t>(n, i0 + per);
    float acc = 0.0f;
    for (int64_t c = i0; c < i1; c += kB) {
        float vv[kB];
#pragma unroll
        for (int j = 0; j < kB; j++) {
            const int64_t i = c + j < i1 ? c + j : i1 - 1;
            vv[j] = vp[svrow[i] + d];
        }
#pragma unroll
        for (int j = 0; j < kB; j++)
            if (c + j < i1) acc = __fadd_rn(acc, __fmul_rn(sprob[c + j], vv[j]));
    }
    part[g][d] = acc;
    __syncthreads();
    if (tid < D) {
        float o = part[0][tid];
#pragma unroll
        for (int q = 1; q < kG; q++) o = __fadd_rn(o, part[q][tid]);
        og[tid] = o;
    }
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
    if (D > 512) return fail(e, SANDY_ERR_UNSUPPORTED, "attention head dimension above 512");
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
    if (a.tk <= kGenStage && env_int("SANDY_ATTN_UNSTAGED", 0) == 0) {
        if (q->dtype == SANDY_BF16) hipLaunchKernelGGL(attention_staged_kernel<BF16>, grid, dim3(256), 0, stream, a);
        else hipLaunchKernelGGL(attention_staged_kernel<F32>, grid, dim3(256), 0, stream, a);
    } else if (q->dtype == SANDY_BF16) {
        hipLaunchKernelGGL(attention_general_kernel<BF16>, grid, dim3(256), 0, stream, a);
    } else {
        hipLaunchKernelGGL(attention_general_kernel<F32>, grid, dim3(256), 0, stream, a);
    }
    SANDY_HIP_TRY(hipGetLastError(), e, "attention launch");
    return ok(e);
}

namespace {

// Shape of a paged decode call, validated (the reference's error wording).
struct PagedCall {
    int64_t B, hq, D, hkv, P, G, max_blocks;
    float sc;
    bool mfma;  // the bf16 MFMA decode kernel takes it
    int64_t q_sb, q_sh, o_sb, o_sh;  // element strides of q / out over batch and head
    // where the pages are: pool mode (block ids through `table` into k_pool /
    // v_pool) or the reference's page tables (k_pages / v_pages)
    const void* k_pool;
    const void* v_pool;
    int64_t page_elems;  // elements from one page to the next (K and V alike)
    int64_t num_pages;
    const int32_t* table;
    int64_t table_stride;
    const uint64_t* k_pages;
    const uint64_t* v_pages;
    int64_t kv_rows_b;
    int64_t tk;  // logical key count (pool mode: max_blocks * P)
};

int check_paged(const SandyTensor* q, const SandyPagedCache* kc, const SandyPagedCache* vc, const SandyTensor* table,
                const SandyTensor* position_offsets, int64_t window, double scale, const SandyTensor* out, Err e,
                PagedCall* c) {
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
    const int64_t dense_page = hkv * kc->page_size * D;
    const int64_t stride = kc->page_stride ? kc->page_stride : dense_page;
    if ((vc->page_stride ? vc->page_stride : dense_page) != stride || stride < dense_page)
        return fail(e, SANDY_ERR_INVALID, "paged attention k and v page strides must match and hold a page");
    if (P <= 0 || (P & (P - 1)) != 0) return fail(e, SANDY_ERR_INVALID, "paged tensor pool page_size must be a power of two");
    if (hq <= 0 || hkv <= 0 || hq % hkv != 0) return fail(e, SANDY_ERR_INVALID, "attention heads must be divisible by kv_heads");
    if (window < 0) return fail(e, SANDY_ERR_INVALID, "attention window must be >= 0");
    if (!same_shape(*q, *out) || out->dtype != q->dtype) return fail(e, SANDY_ERR_INVALID, "attention output shape mismatch");
    if (table->dtype != SANDY_I32 || table->rank != 2 || table->dims[0] != B || table->strides[1] != 1)
        return fail(e, SANDY_ERR_INVALID, "paged attention block table must be [B, max_blocks] int32 with unit inner stride");
    if (!is_index(position_offsets->dtype) || numel(*position_offsets) != B || !contiguous(*position_offsets))
        return fail(e, SANDY_ERR_INVALID, "attention position_offsets length must match batch");
    if (q->strides[3] != 1 || out->strides[3] != 1) return fail(e, SANDY_ERR_UNSUPPORTED, "paged attention needs unit head-dim stride");
    const int64_t G = hq / hkv;
    const bool aligned = ((reinterpret_cast<uintptr_t>(base_ptr(*q)) | reinterpret_cast<uintptr_t>(kc->pool) |
                           reinterpret_cast<uintptr_t>(vc->pool)) & 15u) == 0 &&
                         q->strides[0] % 8 == 0 && q->strides[1] % 8 == 0 && out->strides[0] % 2 == 0 &&
                         out->strides[1] % 2 == 0 && (reinterpret_cast<uintptr_t>(base_ptr(*out)) & 3u) == 0;
    c->B = B;
    c->hq = hq;
    c->D = D;
    c->hkv = hkv;
    c->P = P;
    c->G = G;
    c->max_blocks = table->dims[1];
    c->sc = scale <= 0.0 ? 1.0f / sqrtf(static_cast<float>(D)) : static_cast<float>(scale);
    c->mfma = q->dtype == SANDY_BF16 && (D == 64 || D == 128 || D == 256) && G <= 16 && P % 16 == 0 &&
              table->dims[1] > 0 && table->dims[1] * P <= (1LL << 30) && aligned &&
              env_int("SANDY_PAGED_GENERIC", 0) == 0;
    c->q_sb = q->strides[0];
    c->q_sh = q->strides[1];
    c->o_sb = out->strides[0];
    c->o_sh = out->strides[1];
    c->k_pool = kc->pool;
    c->v_pool = vc->pool;
    c->page_elems = stride;
    c->num_pages = kc->num_pages;
    c->table = static_cast<const int32_t*>(base_ptr(*table));
    c->table_stride = table->strides[0];
    c->k_pages = c->v_pages = nullptr;
    c->kv_rows_b = 0;
    c->tk = table->dims[1] * P;
    return SANDY_OK;
}

// The MFMA decode launch.  `fixed` = nullptr: partials in the grow-only
// device workspace, split merge fused into the decode kernel (arrival
// counters); otherwise partials in the caller-free region `fixed` of
// `fixed_cap` bytes and the two-launch form (decode, then merge), which needs
// no counters and no memory that must start at zero.
int launch_paged_mfma(const PagedCall& c, const SandyTensor* q, const SandyTensor* position_offsets, int64_t window,
                      const SandyTensor* out, uint32_t* errw, char* fixed, size_t fixed_cap, hipStream_t stream,
                      Err e) {
    const int64_t B = c.B, hq = c.hq, D = c.D, hkv = c.hkv, P = c.P, G = c.G, max_blocks = c.max_blocks;
    int status = 0;
    PagedArgs a{};
    a.q = static_cast<const uint16_t*>(base_ptr(*q));
    a.q_sb = c.q_sb;
    a.q_sh = c.q_sh;
    a.out = static_cast<uint16_t*>(base_ptr(*out));
    a.o_sb = c.o_sb;
    a.o_sh = c.o_sh;
    a.k_pool = static_cast<const uint16_t*>(c.k_pool);
    a.v_pool = static_cast<const uint16_t*>(c.v_pool);
    a.page_elems = c.page_elems;
    a.num_pages = c.num_pages;
    a.table = c.table;
    a.table_stride = c.table_stride;
    a.k_pages = c.k_pages;
    a.v_pages = c.v_pages;
    a.kv_rows_b = static_cast<int32_t>(c.kv_rows_b);
    a.tk = c.tk;
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
    a.scale_log2 = c.sc * kLog2e;
    a.batch = static_cast<int32_t>(B);
    a.errw = errw;
    a.fused = fixed ? 0 : env_int("SANDY_PAGED_FUSED_MERGE", 1);
    const int64_t max_keys = std::min(max_blocks * P, c.tk);
    const int nb = D == 64 ? 2 : 1;
    const size_t lds_v = 4 * nb * 16 * (2 * D + 8);
    const size_t lds_r = (4 * G * D + 4 * G * 2) * sizeof(float);
    const size_t lds = std::max(lds_v, lds_r);
    dim3 mgrid(static_cast<unsigned>(hq), static_cast<unsigned>(B));
    void* args[] = {&a};
    // split units of 64*NT keys; about 1024 units at the longest context
    // (measured best with the fused merge: config 3 at 512 keys, config 4 at 1024)
    // (the nearest size on a log scale: a table slightly longer than 4096
    // keys keeps 512-key splits)
    const int64_t forced = env_int("SANDY_PAGED_SPLIT", 0);
    // (D 256: half of it -- 4x the bytes per key; config 4: 512 keys, 122.9 vs 130.4 us at 1024)
    int64_t split = forced > 0 ? forced : (max_keys * B * hkv) / (D == 256 ? 2048 : 1024);
    const int nt = forced > 0 ? (split <= 128 && D == 64 ? 2 : split <= 256 ? 4 : split <= 512 ? 8 : 16)
                              : (split <= 362 ? 4 : split <= 724 ? 8 : 16);
    split = 64 * nt;
    a.split_keys = static_cast<int32_t>(split);
    a.max_splits = static_cast<int32_t>((max_keys + split - 1) / split);
    const int64_t units = static_cast<int64_t>(a.max_splits) * hkv * B;
    if (units > (1LL << 26)) return fail(e, SANDY_ERR_UNSUPPORTED, "paged attention batch too large");
    const size_t slots = static_cast<size_t>(B * hq * a.max_splits);
    const size_t ws_bytes = slots * (D + 2) * sizeof(float);
    char* ws = fixed;
    if (fixed) {
        if (ws_bytes > fixed_cap)
            return fail(e, SANDY_ERR_UNSUPPORTED,
                        "paged attention without allocation needs %zu bytes of split partials; its fixed scratch holds %zu",
                        ws_bytes, fixed_cap);
    } else {
        ws = static_cast<char*>(device_workspace(0, ws_bytes, stream, e, &status));
        if (status) return status;
        if (a.fused) {
            a.counters = static_cast<uint32_t*>(
                device_counters(0, static_cast<size_t>(B * hkv) * sizeof(uint32_t), stream, e, &status));
            if (status) return status;
        }
    }
    a.ws_o = reinterpret_cast<float*>(ws);
    a.ws_ml = reinterpret_cast<float*>(ws + slots * D * sizeof(float));
    // work units numbered over the active splits; whole splits first when the
    // grid (active and idle units) exceeds two rounds of resident workgroups,
    // where the active ones alone take more than one (config 4: 121.2-122.8 ->
    // 119.0-120.2 us); config 3's 640 active of 1024 units fit one round and
    // keep sequence order (23.5-23.9 against 23.6-23.9 with whole splits first)
    const bool lpt = units > 2 * resident_workgroups(units_kernel(static_cast<int>(D), nt), lds);
    // grids of at most one workgroup a CU with no window (batch-1 decode
    // steps): the static schedule, block ids requested with the position
    // (TinyLlama batch-1 step 1044.1-1045.4 -> 1038.3-1040.4 us)
    const bool stat = window == 0 && units <= device_cu_count();
    SANDY_HIP_TRY(hipLaunchKernel(stat ? static_kernel(static_cast<int>(D), nt) : units_kernel(static_cast<int>(D), nt, lpt),
                                  dim3(static_cast<unsigned>(units)), dim3(256), args, lds, stream),
                  e, "paged attention launch");
    const void* mfn = D == 64 ? reinterpret_cast<const void*>(&paged_decode_units_merge_kernel<64>)
                    : D == 128 ? reinterpret_cast<const void*>(&paged_decode_units_merge_kernel<128>)
                               : reinterpret_cast<const void*>(&paged_decode_units_merge_kernel<256>);
    if (!a.fused)
        SANDY_HIP_TRY(hipLaunchKernel(mfn, mgrid, dim3(64), args, 0, stream), e, "paged attention merge launch");
    SANDY_HIP_TRY(hipGetLastError(), e, "paged attention launch");
    return ok(e);
}

} // namespace

extern "C" int sandy_hip_paged_attention(const SandyTensor* q, const SandyPagedCache* kc, const SandyPagedCache* vc,
                                         const SandyTensor* table, const SandyTensor* position_offsets,
                                         int64_t window, double scale, const SandyTensor* out, void* stream_,
                                         char* err, size_t err_cap) {
    Err e{err, err_cap};
    hipStream_t stream = static_cast<hipStream_t>(stream_);
    PagedCall c{};
    int status = check_paged(q, kc, vc, table, position_offsets, window, scale, out, e, &c);
    if (status) return status;
    if (c.B == 0) return ok(e);
    uint32_t* errw = device_error_word(e, &status);
    if (status) return status;
    if (c.mfma) return launch_paged_mfma(c, q, position_offsets, window, out, errw, nullptr, 0, stream, e);
    const int64_t B = c.B, hq = c.hq, D = c.D, hkv = c.hkv, P = c.P, max_blocks = c.max_blocks;
    const float sc = c.sc;
    if (D > 512) return fail(e, SANDY_ERR_UNSUPPORTED, "attention head dimension above 512");
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
    a.page_elems = c.page_elems;
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
    // fp32 steps of the common head dims: the decode kernel (16-byte rows)
    const bool dec = q->dtype == SANDY_F32 && a.tk <= kGenStage && (D == 32 || D == 64 || D == 128 || D == 256) &&
                     (c.page_elems % 4) == 0 && ((reinterpret_cast<uintptr_t>(kc->pool) |
                                                  reinterpret_cast<uintptr_t>(vc->pool)) & 15u) == 0 &&
                     env_int("SANDY_ATTN_UNSTAGED", 0) == 0;
    if (dec) {
        switch (D) {
            case 32: hipLaunchKernelGGL(attention_decode_f32_kernel<32>, grid, dim3(256), 0, stream, a); break;
            case 64: hipLaunchKernelGGL(attention_decode_f32_kernel<64>, grid, dim3(256), 0, stream, a); break;
            case 128: hipLaunchKernelGGL(attention_decode_f32_kernel<128>, grid, dim3(256), 0, stream, a); break;
            default: hipLaunchKernelGGL(attention_decode_f32_kernel<256>, grid, dim3(256), 0, stream, a); break;
        }
    } else if (a.tk <= kGenStage && env_int("SANDY_ATTN_UNSTAGED", 0) == 0) {
        if (q->dtype == SANDY_BF16) hipLaunchKernelGGL(attention_staged_kernel<BF16>, grid, dim3(256), 0, stream, a);
        else hipLaunchKernelGGL(attention_staged_kernel<F32>, grid, dim3(256), 0, stream, a);
    } else if (q->dtype == SANDY_BF16) {
        hipLaunchKernelGGL(attention_general_kernel<BF16>, grid, dim3(256), 0, stream, a);
    } else {
        hipLaunchKernelGGL(attention_general_kernel<F32>, grid, dim3(256), 0, stream, a);
    }
    SANDY_HIP_TRY(hipGetLastError(), e, "paged attention launch");
    return ok(e);
}

// AttentionKernelOp with the reference's own paged K/V (a CudaDeviceBufferView
// with paged = true: page table, logical shape, page size and count).  Same
// validation and semantics as sandy_hip_attention on the dense tensors the
// pages hold; decode steps (Tq = 1) of the bf16 MFMA shapes take the paged
// decode kernel in page-table mode, everything else the general kernel.
extern "C" int sandy_hip_attention_paged_view(const SandyTensor* q, const SandyPagedView* k, const SandyPagedView* v,
                                              const SandyTensor* position_offsets, int64_t window, double scale,
                                              const SandyTensor* out, void* stream_, char* err, size_t err_cap) {
    Err e{err, err_cap};
    hipStream_t stream = static_cast<hipStream_t>(stream_);
    if (!valid_rank(q) || !valid_rank(out) || !k || !v) return fail(e, SANDY_ERR_INVALID, "attention tensor rank out of range");
    if (!k->pages || !v->pages) return fail(e, SANDY_ERR_INVALID, "attention paged view requires a page table");
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
    if (D > 512) return fail(e, SANDY_ERR_UNSUPPORTED, "attention head dimension above 512");
    const int64_t P = k->page_size;
    if (P <= 0 || (P & (P - 1)) != 0 || v->page_size != P)
        return fail(e, SANDY_ERR_INVALID, "paged tensor pool page_size must be a power of two");
    if (tk < 0 || k->page_count < (tk + P - 1) / P || v->page_count < (tk + P - 1) / P)
        return fail(e, SANDY_ERR_INVALID, "paged tensor page count does not cover its logical shape");
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
    const float sc = scale <= 0.0 ? 1.0f / sqrtf(static_cast<float>(D)) : static_cast<float>(scale);
    const int64_t q_sb = rank == 4 ? q->strides[0] : 0, q_sh = q->strides[o];
    const int64_t o_sb = rank == 4 ? out->strides[0] : 0, o_sh = out->strides[o];
    const int64_t G = hq / hkv;
    const bool aligned = (reinterpret_cast<uintptr_t>(base_ptr(*q)) & 15u) == 0 && q_sb % 8 == 0 && q_sh % 8 == 0 &&
                         o_sb % 2 == 0 && o_sh % 2 == 0 && (reinterpret_cast<uintptr_t>(base_ptr(*out)) & 3u) == 0 &&
                         q->strides[rank - 1] == 1 && out->strides[rank - 1] == 1;
    const bool mfma = tq == 1 && position_offsets && q->dtype == SANDY_BF16 && (D == 64 || D == 128 || D == 256) &&
                      G <= 16 && P % 16 == 0 && tk > 0 && tk <= (1LL << 30) && aligned &&
                      env_int("SANDY_PAGED_GENERIC", 0) == 0;
    if (mfma) {
        PagedCall c{};
        c.B = B;
        c.hq = hq;
        c.D = D;
        c.hkv = hkv;
        c.P = P;
        c.G = G;
        c.max_blocks = (tk + P - 1) / P;
        c.sc = sc;
        c.mfma = true;
        c.q_sb = q_sb;
        c.q_sh = q_sh;
        c.o_sb = o_sb;
        c.o_sh = o_sh;
        c.k_pages = static_cast<const uint64_t*>(k->pages);
        c.v_pages = static_cast<const uint64_t*>(v->pages);
        c.kv_rows_b = rank == 4 ? hkv : 0;
        c.tk = tk;
        return launch_paged_mfma(c, q, position_offsets, window, out, errw, nullptr, 0, stream, e);
    }
    GenArgs a{};
    auto fill4 = [&](const SandyTensor* t, int64_t* st) {
        if (rank == 4) for (int i = 0; i < 4; i++) st[i] = t->strides[i];
        else { st[0] = 0; for (int i = 0; i < 3; i++) st[i + 1] = t->strides[i]; }
    };
    a.q = base_ptr(*q);
    fill4(q, a.qs);
    a.out = base_ptr(*out);
    fill4(out, a.os);
    a.k = nullptr;  // page-table mode: offsets are absolute element addresses
    a.v = nullptr;
    a.dt = q->dtype;
    a.paged = 1;
    a.page_size = P;
    a.k_pages = static_cast<const uint64_t*>(k->pages);
    a.v_pages = static_cast<const uint64_t*>(v->pages);
    a.kv_rows_b = rank == 4 ? hkv : 0;
    a.max_blocks = (tk + P - 1) / P;
    a.pos = position_offsets ? base_ptr(*position_offsets) : nullptr;
    a.pos_dt = position_offsets ? position_offsets->dtype : SANDY_I64;
    a.hq = static_cast<int32_t>(hq);
    a.hkv = static_cast<int32_t>(hkv);
    a.tq = static_cast<int32_t>(tq);
    a.tk = tk;
    a.d = D;
    a.window = window;
    a.scale = sc;
    const size_t sbytes = static_cast<size_t>(B * hq * tq * std::max<int64_t>(tk, 1)) * sizeof(float);
    a.scores = static_cast<float*>(device_workspace(1, sbytes, stream, e, &status));
    if (status) return status;
    a.errw = errw;
    dim3 grid(static_cast<unsigned>(tq), static_cast<unsigned>(hq), static_cast<unsigned>(B));
    if (a.tk <= kGenStage && env_int("SANDY_ATTN_UNSTAGED", 0) == 0) {
        if (q->dtype == SANDY_BF16) hipLaunchKernelGGL(attention_staged_kernel<BF16>, grid, dim3(256), 0, stream, a);
        else hipLaunchKernelGGL(attention_staged_kernel<F32>, grid, dim3(256), 0, stream, a);
    } else if (q->dtype == SANDY_BF16) {
        hipLaunchKernelGGL(attention_general_kernel<BF16>, grid, dim3(256), 0, stream, a);
    } else {
        hipLaunchKernelGGL(attention_general_kernel<F32>, grid, dim3(256), 0, stream, a);
    }
    SANDY_HIP_TRY(hipGetLastError(), e, "attention launch");
    return ok(e);
}

namespace {

// Scratch of sandy_hip_paged_attention_noalloc: the (O, max, sum) split
// partials of its two-launch decode, at most kNoAllocScratch bytes (config 4
// -- 64 sequences of up to 8192 keys, 8 q heads, D 256 -- needs 4.2 MB;
// config 3 2.2 MB).  Each GPU the library runs on holds its own copy until
// the process ends.  Host code never passes the name: it uses the address
// hipGetSymbolAddress gives for the current device (scratch_address).
constexpr size_t kNoAllocScratch = 8u << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratch];

constexpr int kScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch[kScratchDevices] = {};

int scratch_address(Err e, char** out) {
    int dev = 0;
    SANDY_HIP_TRY(hipGetDevice(&dev), e, "hipGetDevice");
    if (dev < 0 || dev >= kScratchDevices) return fail(e, SANDY_ERR_HIP, "device ordinal %d out of range", dev);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch[dev]) {
        void* p = nullptr;
        const hipError_t st = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (st != hipSuccess) return fail(e, SANDY_ERR_HIP, "paged attention scratch address: %s", hipGetErrorString(st));
        g_scratch[dev] = p;
    }
    *out = static_cast<char*>(g_scratch[dev]);
    return SANDY_OK;
}

} // namespace

// The no-allocation variant of sandy_hip_paged_attention (bf16 MFMA decode
// shapes only): its split partials live in the file-scope `scratch` above,
// so it calls no allocator, and the split merge runs as a second launch, so
// nothing in the scratch has to start at zero.  Calls overlapping on one GPU
// share the scratch and race.
extern "C" int sandy_hip_paged_attention_noalloc(const SandyTensor* q, const SandyPagedCache* kc,
                                                 const SandyPagedCache* vc, const SandyTensor* table,
                                                 const SandyTensor* position_offsets, int64_t window, double scale,
                                                 const SandyTensor* out, void* stream_, char* err, size_t err_cap) {
    Err e{err, err_cap};
    hipStream_t stream = static_cast<hipStream_t>(stream_);
    PagedCall c{};
    int status = check_paged(q, kc, vc, table, position_offsets, window, scale, out, e, &c);
    if (status) return status;
    if (!c.mfma)
        return fail(e, SANDY_ERR_UNSUPPORTED,
                    "paged attention without allocation takes bf16 q with head dim 64, 128 or 256, at most 16 q heads "
                    "per kv head, 16-row pages and 16-byte aligned operands");
    if (c.B == 0) return ok(e);
    uint32_t* errw = device_error_word(e, &status);
    if (status) return status;
    char* ws = nullptr;
    status = scratch_address(e, &ws);
    if (status) return status;
    return launch_paged_mfma(c, q, position_offsets, window, out, errw, ws, kNoAllocScratch, stream, e);
}
