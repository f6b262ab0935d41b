// gemm.h -- the decode GEMM (gemm_waves_kernel) and the types shared by the
// matmul translation units: matmul.hip (every other form and the host
// dispatch) and matmul_norm.hip (the RMSNorm-prologue instantiations, a
// translation unit of their own so the two halves compile in parallel).
#pragma once
#include "common.h"

namespace sandy_hip {
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

// Element offsets of batch index b in each operand.  For each output batch
// dim d (innermost first): coordinate c = b mod dims[d]; an operand adds
// (c / div[d]) * stride[d] (stride 0 where it broadcasts a size-1 or absent
// dim; div = out dim / operand dim for a grouped dim).
struct BatchMap {
    int32_t rank;
    int64_t dims[SANDY_HIP_MAX_RANK];
    int64_t l_stride[SANDY_HIP_MAX_RANK], l_div[SANDY_HIP_MAX_RANK];
    int64_t r_stride[SANDY_HIP_MAX_RANK], r_div[SANDY_HIP_MAX_RANK];
};

__device__ __forceinline__ void batch_offsets(const BatchMap& m, int64_t b, int64_t& lo, int64_t& ro) {
    lo = 0;
    ro = 0;
    for (int d = m.rank - 1; d >= 0; d--) {
        const int64_t c = b % m.dims[d];
        b /= m.dims[d];
        lo += (c / m.l_div[d]) * m.l_stride[d];
        ro += (c / m.r_div[d]) * m.r_stride[d];
    }
}

// q/k/v epilogue of the decode GEMM (sandy_hip_device_matmul_qkv): row r of
// the product is sequence r's q/k/v row.  Its q and k columns are RoPE-rotated
// (q into q_out [M, hq, d], k appended to the sequence's K pages) and its v
// columns appended to the V pages, at row pos[r] of the sequence, whose K and
// V lengths become pos[r] + 1.  With split-half RoPE the weight's q and k rows
// come pair-ordered within each head (rows i and i + d / 2 adjacent), so both
// values of a rotation pair sit in lanes l and l ^ 1 of an MFMA tile.
constexpr int kQkvMaxPairs = 128;
constexpr int kQkvMaxRows = 64;
struct QkvRope {
    uint16_t* q_out;
    char* k_pages;
    char* v_pages;
    const int32_t* k_table;
    const int32_t* v_table;
    int32_t* k_len;
    int32_t* v_len;
    int64_t page_bytes;
    int32_t k_max_blocks, v_max_blocks, page_shift, hq, hkv, d, split_half, pos_dt;
    const void* pos;
    uint32_t* errw;
    // [row tiles] arrivals (zero between launches): the workgroup that counts
    // itself in last advances the row tile's lengths, after every workgroup
    // has read them (a tile that read an advanced length would take a valid
    // append for a stale position)
    uint32_t* arrivals;
    int32_t kv_arrivals;  // workgroups per row tile whose columns include k or v
    float denom[kQkvMaxPairs];  // theta^(2i / d), host float powf
    int32_t k_slots[kQkvMaxRows];
    int32_t v_slots[kQkvMaxRows];
};

struct GemmArgs {
    const uint16_t* a;     // [.., M, K]
    const uint16_t* w;     // [.., N, K]
    const uint16_t* bias;  // [N] or null
    uint16_t* out;         // [batch, M, N]
    int64_t M, N, K;
    int32_t col_tiles, row_tiles, splits, split_chunks;
    float* part;           // [tiles, splits, 4 waves, RT * CT * 64 lanes * 4]
    uint32_t* counters;    // [tiles] arrivals (zero between launches)
    BatchMap bm;
    int32_t glu;           // 0: plain; 1 / 2: gated SiLU / GELU epilogue (weight rows interleaved gate, up)
    // residual epilogue (decode GEMM): out = bf16(resid + bf16(product)), and
    // per (row, 16-column group) float64 sums of squares of out in rsq_out
    // [M, rsq_parts] (rsq_parts = ceil(N / 16)); resid null: plain epilogue
    const uint16_t* resid;
    double* rsq_out;
    int64_t rsq_parts;
    // RMSNorm prologue (decode GEMM, NORM kernels): the A operand is
    // bf16(a * inv * norm_w) with inv = 1 / sqrt(float(sum / K) + eps) and sum
    // the row's rsq_in partials [M, rsq_in_parts]
    const double* rsq_in;
    int64_t rsq_in_parts;
    const uint16_t* norm_w;
    float eps;
    QkvRope qr;
};

// Gated activation of one bf16-rounded (gate, up) pair with the scalar DAGs
// of src/ir/BuiltinLowering.cpp:116-158 in their node order (silu(g) * up,
// gelu(g) * up), fp32 arithmetic without contraction -- what the generated
// element-wise group computes from the two GEMM outputs.
__device__ __forceinline__ float glu_pair(int kind, float gv, float uv) {
    if (kind == 1) {
        const float h = __fmul_rn(0.5f, gv);
        return __fmul_rn(sandy_silu_half(h), uv);
    }
    const float h = __fmul_rn(0.5f, gv);
    const float x3 = __fmul_rn(__fmul_rn(gv, gv), gv);
    const float inner = __fadd_rn(gv, __fmul_rn(0.044715f, x3));
    const float t = sandy_tanh(__fmul_rn(0.7978845608028654f, inner));
    return __fmul_rn(__fmul_rn(h, __fadd_rn(1.0f, t)), uv);
}


// Decode-shaped products (a few dozen rows against megabytes of weights):
// workgroup = 16 * CT output columns x 16 * RT rows; its four waves take
// consecutive quarters of the workgroup's K range and run independently --
// no workgroup barrier inside the K loop -- so each wave keeps Q chunks of
// its weight rows in flight on its own.  A wave loads its 16 * CT weight rows
// as whole 128-byte lines into a private, swizzled, double-buffered LDS tile
// (read back in MFMA layout) and its activation rows straight into MFMA
// A-operand registers (they are L2-resident; every workgroup reads them).
// The K loop is straight-line over CPS chunks so every register slot is
// statically named and each LDS write waits only for its own chunk.  The
// four partial accumulators are summed in wave order through LDS; when the
// grid also splits K across workgroups, the last-arriving workgroup of each
// tile sums the splits' fp32 partials in split order (deterministic).
// NT: the weight stream is read with the non-temporal policy (each line is
// used once per launch); off where another workgroup's re-read of the same
// weights should still find them in L2 (row tiles that do not run together)
template <int RT, int CT, int Q, int CPS, int OCC, bool NORM = false, bool ROPE = false, bool NT = false>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(OCC))) void gemm_waves_kernel(GemmArgs g) {
    constexpr int kWTile = 16 * CT * 128;
    // activation rows staged through LDS as whole lines (XL) for tiles of up to
    // 32 columns, where they are half the bytes a wave loads; the 64-column
    // tiles load them straight into A registers (measured: o projection
    // 6.6 -> 5.8 us, q/k/v 7.9 -> 7.3, down 13.6 -> 12.7; lm-head 29.4 -> 33.3)
    constexpr bool XL = CT <= 2;
    constexpr int kXTile = XL ? 16 * RT * 128 : 0;  // one chunk of the activation rows
    constexpr int kAcc = RT * CT * 64 * 16;  // one wave's accumulators, bytes
    // per wave: double-buffered weight tile, one activation tile (a wave's LDS
    // reads of chunk c are issued before its writes of chunk c + 1, and one
    // wave's LDS operations complete in order)
    constexpr int kLds = 4 * (2 * kWTile + kXTile) > 3 * kAcc ? 4 * (2 * kWTile + kXTile) : 3 * kAcc;
    __shared__ __attribute__((aligned(16))) unsigned char lds[kLds];
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int ct = static_cast<int>(blockIdx.x) / g.splits;
    const int split = static_cast<int>(blockIdx.x) % g.splits;
    const int64_t r0 = static_cast<int64_t>(blockIdx.y) * 16 * RT;
    const int64_t bz = blockIdx.z;
    int64_t lo, ro;
    batch_offsets(g.bm, bz, lo, ro);
    const int64_t M = g.M, N = g.N, K = g.K;
    const int64_t n0 = static_cast<int64_t>(ct) * 16 * CT;
    unsigned char* wt = lds + wave * (2 * kWTile + kXTile);
    unsigned char* xt = wt + 2 * kWTile;
    auto swz = [](int row, int piece) { return row * 128 + ((piece ^ ((row >> 1) & 7)) << 4); };
    const int ksteps = static_cast<int>(K / 32);
    const int chunks = (ksteps + 1) / 2;
    const int wg_begin = split * g.split_chunks;
    const int wg_end = min(chunks, wg_begin + g.split_chunks);
    const int c_begin = min(wg_end, wg_begin + wave * CPS);
    const int c_end = min(wg_end, c_begin + CPS);

    const int64_t wrows = min<int64_t>(16 * CT, N - n0);
    const __amdgpu_buffer_rsrc_t wres = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(g.w + ro + n0 * K), 0, static_cast<int>(wrows * K * 2), 0x00020000);
    const int64_t xrows = min<int64_t>(16 * RT, M - r0);
    const __amdgpu_buffer_rsrc_t xres = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(g.a + lo + r0 * K), 0, static_cast<int>(xrows * K * 2), 0x00020000);
    const int wlane = static_cast<int>((lane >> 3) * K * 2 + (lane & 7) * 16);
    const int wstep = static_cast<int>(8 * K * 2);
    const int wbase[2] = {swz(lane >> 3, lane & 7), swz(8 + (lane >> 3), lane & 7) - 1024};
    int raddr[2][CT];
#pragma unroll
    for (int u = 0; u < 2; u++)
#pragma unroll
        for (int c = 0; c < CT; c++) raddr[u][c] = swz(16 * c + (lane & 15), 4 * u + (lane >> 4));
    // A operand of tile t, k-step u: row 16 t + lane % 16, 16-byte piece 4 u + lane / 16 -- in the
    // activation tile (XL) or in global memory
    int aaddr[2][RT];
#pragma unroll
    for (int u = 0; u < 2; u++)
#pragma unroll
        for (int t = 0; t < RT; t++)
            aaddr[u][t] = XL ? swz(16 * t + (lane & 15), 4 * u + (lane >> 4))
                             : static_cast<int>((16 * t + (lane & 15)) * K * 2 + (4 * u + (lane >> 4)) * 16);

    f32x4_t acc[RT][CT];
#pragma unroll
    for (int t = 0; t < RT; t++)
#pragma unroll
        for (int c = 0; c < CT; c++) acc[t][c] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    // RMSNorm prologue, part 1: the partial sums of squares of the workgroup's
    // rows are requested before the K stream (their wait does not cover it)
    constexpr int kRows = 16 * RT;
    constexpr int kTpr = 256 / kRows;  // threads per row
    __shared__ float inv_s[kRows];
    // the first 16 partials of this thread, all requested before the weight
    // stream (clamped addresses; unused values dropped by a select when summed)
    // as many as a 2048-wide row's 128 partials need (longer rows sum the rest
    // in a loop)
    constexpr int kPq = NORM ? kRows / 2 : 1;
    double pv[kPq];
    const int64_t prow = NORM ? min<int64_t>(r0 + tid / kTpr, M - 1) : 0;
    if constexpr (NORM) {
        const int64_t parts = g.rsq_in_parts;
#pragma unroll
        for (int q = 0; q < kPq; q++) {
            const int64_t pp = q * kTpr + tid % kTpr;
            pv[q] = g.rsq_in[prow * parts + (pp < parts ? pp : parts - 1)];
        }
    }
    // residual epilogue: this lane's residual values, requested now (packed
    // bf16 pairs: rows 4 (lane / 16) + {0, 1} and {2, 3} of tile t, column c)
    uint32_t rres[RT][CT][2];
    if (g.resid) {
#pragma unroll
        for (int t = 0; t < RT; t++)
#pragma unroll
            for (int c = 0; c < CT; c++) {
                const int64_t nc = min<int64_t>(n0 + 16 * c + (lane & 15), N - 1);
                uint32_t h[4];
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int64_t rr = min<int64_t>(r0 + 16 * t + 4 * (lane >> 4) + i, M - 1);
                    h[i] = g.resid[bz * M * N + rr * N + nc];
                }
                rres[t][c][0] = h[0] | (h[1] << 16);
                rres[t][c][1] = h[2] | (h[3] << 16);
            }
    }
    // q/k/v epilogue (wave 0 emits the tile): each lane's rows' positions and
    // slots, and its columns' angle denominators, requested now; the block ids
    // and lengths that depend on them go out once the first weight chunks are
    // in flight.  32-bit index math (a 64-bit division is a long software loop)
    int32_t qpos[RT][4], qks[RT][4], qvs[RT][4], qkb[RT][4], qvb[RT][4], qkl[RT][4], qvl[RT][4];
    float qden[CT], qsn[RT][4][CT], qcs[RT][4][CT];
    if constexpr (ROPE) {
        // every wave requests them (a wave-0-only branch makes the compiler
        // copy the results at the join, waiting for each load there)
#pragma unroll
        for (int t = 0; t < RT; t++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int rr = min(static_cast<int>(r0) + 16 * t + 4 * (lane >> 4) + i, static_cast<int>(M) - 1);
                qpos[t][i] = static_cast<int32_t>(load_index(g.qr.pos, g.qr.pos_dt, rr));
                qks[t][i] = g.qr.k_slots[rr];
                qvs[t][i] = g.qr.v_slots[rr];
            }
#pragma unroll
        for (int c = 0; c < CT; c++) {
            const uint32_t nc = static_cast<uint32_t>(min<int64_t>(n0 + 16 * c + (lane & 15), N - 1));
            qden[c] = g.qr.denom[(nc % static_cast<uint32_t>(g.qr.d)) >> 1];
        }
    }
    // norm weights per chunk: XL normalises the activation pieces it stages
    // (one 16-byte piece per lane), otherwise the A operands (two)
    uint4 wv[Q][2 * CT], xv[Q][2 * RT], nv[NORM ? Q : 1][XL ? 1 : 2];
    const __amdgpu_buffer_rsrc_t nres = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(NORM ? g.norm_w : g.w), 0, NORM ? static_cast<int>(K * 2) : 0, 0x00020000);
    // clamped re-reads past this wave's range: L2 hits, never multiplied
    auto load = [&](int ch, int slot) {
        const int kb = max(0, min(ch, c_end - 1)) * 128;
#pragma unroll
        for (int i = 0; i < 2 * CT; i++)
            wv[slot][i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(wres, wlane + i * wstep + kb, 0, NT ? 2 : 0));
        // XL: the activation rows as whole lines too (8 rows x 128 bytes per
        // instruction), staged through LDS like the weights; otherwise the
        // A operands themselves (half of 16 lines per instruction)
#pragma unroll
        for (int i = 0; i < 2 * RT; i++)
            xv[slot][i] = __builtin_bit_cast(
                uint4, __builtin_amdgcn_raw_buffer_load_b128(
                           xres, XL ? wlane + i * wstep + kb : aaddr[i & 1][i >> 1] + kb, 0, 0));
        if constexpr (NORM && XL)
            nv[slot][0] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(nres, (lane & 7) * 16 + kb, 0, 0));
        else if constexpr (NORM)
#pragma unroll
            for (int u = 0; u < 2; u++)
                nv[slot][u] = __builtin_bit_cast(uint4,
                                                 __builtin_amdgcn_raw_buffer_load_b128(nres, (4 * u + (lane >> 4)) * 16 + kb, 0, 0));
    };
    float inv[RT];  // RMSNorm prologue: 1 / rms of this lane's A-operand rows
    float invx[2 * RT];  // (XL) 1 / rms of the rows whose pieces this lane stages
    // y = bf16(x * inv * w): the RMSNorm kernel's operation order, rounded once
    // to nearest even by gfx950's v_cvt_pk_bf16_f32 (f32_to_bf16's rounding)
    auto normed = [&](const uint4& xr, const uint4& wr, float iv) -> uint4 {
        const uint32_t xs[4] = {xr.x, xr.y, xr.z, xr.w}, ws[4] = {wr.x, wr.y, wr.z, wr.w};
        uint32_t o[4];
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const float lo = __fmul_rn(__fmul_rn(__uint_as_float(xs[q] << 16), iv), __uint_as_float(ws[q] << 16));
            const float hi = __fmul_rn(__fmul_rn(__uint_as_float(xs[q] & 0xffff0000u), iv),
                                       __uint_as_float(ws[q] & 0xffff0000u));
            o[q] = __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{lo, hi}, bf16x2_t));
        }
        return make_uint4(o[0], o[1], o[2], o[3]);
    };
    auto store = [&](int slot, int buf) {
#pragma unroll
        for (int i = 0; i < 2 * CT; i++) *reinterpret_cast<uint4*>(wt + buf * kWTile + wbase[i & 1] + i * 1024) = wv[slot][i];
        // (NORM) normalised as they are staged: this VALU work overlaps the
        // previous chunk's MFMAs instead of sitting in front of the next ones
        if constexpr (XL)
#pragma unroll
            for (int i = 0; i < 2 * RT; i++)
                *reinterpret_cast<uint4*>(xt + wbase[i & 1] + i * 1024) =
                    NORM ? normed(xv[slot][i], nv[slot][0], invx[i]) : xv[slot][i];
    };
    // the second k-step of a half chunk (odd K / 32) is skipped, so the
    // registers past K never reach an MFMA
    auto mma = [&](int slot, int buf, int ch) {
#pragma unroll
        for (int u = 0; u < 2; u++) {
            if (u == 1 && 2 * ch + 1 >= ksteps) break;
            uint4 av[RT];
#pragma unroll
            for (int t = 0; t < RT; t++) {
                const uint4 xa = XL ? *reinterpret_cast<const uint4*>(xt + aaddr[u][t]) : xv[slot][2 * t + u];
                if constexpr (NORM && !XL) av[t] = normed(xa, nv[slot][u], inv[t]);
                else av[t] = xa;
            }
#pragma unroll
            for (int c = 0; c < CT; c++) {
                const uint4 bv = *reinterpret_cast<const uint4*>(wt + buf * kWTile + raddr[u][c]);
#pragma unroll
                for (int t = 0; t < RT; t++)
                    acc[t][c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, av[t]),
                                                                        __builtin_bit_cast(bf16x8_t, bv), acc[t][c],
                                                                        0, 0, 0);
            }
        }
    };
    // q/k/v: column tiles that hold a k or v column (the first of them, kv_first,
    // reports the rows' position and block errors); q-only tiles store no cache
    // rows and read no block ids or lengths
    const int64_t q_cols = ROPE ? static_cast<int64_t>(g.qr.hq) * g.qr.d : 0;
    const bool kv_tile = ROPE && n0 + 16 * CT > q_cols;
    const int kv_first = static_cast<int>(q_cols / (16 * CT));
    auto rope_ids = [&]() {
        // slot -> block id of the row's page and the slot's lengths, requested
        // unconditionally (clamped indices; a block index past the table is
        // flagged in the epilogue, the loaded id ignored)
        if (!kv_tile) {
#pragma unroll
            for (int t = 0; t < RT; t++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    qkb[t][i] = qvb[t][i] = 0;
                    qkl[t][i] = qvl[t][i] = qpos[t][i];
                }
        }
#pragma unroll
        for (int t = 0; t < RT; t++)
#pragma unroll
            for (int i = 0; i < 4 && kv_tile; i++) {
                const int32_t bi = max(qpos[t][i], 0) >> g.qr.page_shift;
                const int32_t ks = qks[t][i], vs = qvs[t][i];
                qkb[t][i] = g.qr.k_table[ks * g.qr.k_max_blocks + min(bi, g.qr.k_max_blocks - 1)];
                qvb[t][i] = g.qr.v_table[vs * g.qr.v_max_blocks + min(bi, g.qr.v_max_blocks - 1)];
                qkl[t][i] = g.qr.k_len[ks];
                qvl[t][i] = g.qr.v_len[vs];
            }
        // the rotation angles of this lane's (row, column) pairs, while the
        // first chunks are in flight (the epilogue only multiplies)
#pragma unroll
        for (int t = 0; t < RT; t++)
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int c = 0; c < CT; c++)
                    rope_sincos(static_cast<float>(max(qpos[t][i], 0)) / qden[c], &qsn[t][i][c], &qcs[t][i][c]);
    };
#pragma unroll
    for (int s = 0; s < Q; s++) load(c_begin + s, s);
    if constexpr (NORM) {
        // RMSNorm prologue, part 2 (the first chunks' loads are in flight): the
        // row's sum over its partials, then the RMSNorm kernel's inverse
        // (acc / cols in double, to float, + eps)
        double rsq = 0.0;
        const int64_t parts = g.rsq_in_parts;
#pragma unroll
        for (int q = 0; q < kPq; q++) rsq += q * kTpr + tid % kTpr < parts ? pv[q] : 0.0;
        for (int64_t pp = kPq * kTpr + tid % kTpr; pp < parts; pp += kTpr) rsq += g.rsq_in[prow * parts + pp];
        rsq = group_sum<kTpr>(rsq);
        if (tid % kTpr == 0)
            inv_s[tid / kTpr] = 1.0f / sqrtf(static_cast<float>(rsq / static_cast<double>(K)) + g.eps);
        __syncthreads();
#pragma unroll
        for (int t = 0; t < RT; t++) inv[t] = inv_s[16 * t + (lane & 15)];
#pragma unroll
        for (int i = 0; i < 2 * RT; i++) invx[i] = inv_s[(lane >> 3) + 8 * i];
    }
    // q/k/v: a workgroup whose columns include k or v (only those store into
    // the caches, so only those read the lengths) counts itself in once it has
    // its rows' lengths (the values are used before the atomic, so the loads
    // have returned); the one that arrives last writes the advanced lengths at
    // its end.  The count goes out inside the K loop, after the chunk that was
    // requested behind the lengths, so its round trip overlaps the remaining
    // chunks.
    uint32_t arrive = 0;
    auto count_in = [&]() {
        if (tid == 0 && kv_tile) {
            int32_t dep = 0;
#pragma unroll
            for (int t = 0; t < RT; t++)
#pragma unroll
                for (int i = 0; i < 4; i++) dep += qkl[t][i] + qvl[t][i];
            asm volatile("" ::"v"(dep));
            arrive = __hip_atomic_fetch_add(g.qr.arrivals + blockIdx.y, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    };
    constexpr int kCountAt = Q + 1 < CPS ? Q + 1 : CPS - 1;
    store(0, 0);
#pragma unroll
    for (int u = 0; u < CPS; u++) {
        const int c = c_begin + u;
        if (c < c_end) mma(u % Q, u & 1, c);
        if (c + 1 < c_end) store((u + 1) % Q, (u + 1) & 1);
        load(c + Q, u % Q);
        // q/k/v epilogue ids after the first chunk: the positions they index by
        // arrived with it, so nothing waits and every first chunk went out first
        if constexpr (ROPE) {
            if (u == 0) rope_ids();
            if (u == kCountAt) count_in();
        }
    }
    // the lengths of this row tile's rows advance to pos + 1 where the row was
    // appended (position at the length, pages present), by the last arrival
    auto rope_lengths = [&]() {
        if (!kv_tile || __builtin_amdgcn_readfirstlane(arrive) != static_cast<uint32_t>(g.qr.kv_arrivals - 1)) return;
        if (tid == 0) __hip_atomic_store(g.qr.arrivals + blockIdx.y, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if ((lane & 15) != 0) return;
        const int32_t kmax = g.qr.k_max_blocks, vmax = g.qr.v_max_blocks;
#pragma unroll
        for (int t = 0; t < RT; t++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int rr = static_cast<int>(r0) + 16 * t + 4 * (lane >> 4) + i;
                const int32_t pos = qpos[t][i];
                if (rr >= M || pos < 0 || qkl[t][i] != pos || qvl[t][i] != pos) continue;
                const int32_t bi = pos >> g.qr.page_shift;
                if (bi >= kmax || bi >= vmax || qkb[t][i] < 0 || qvb[t][i] < 0) continue;
                g.qr.k_len[qks[t][i]] = pos + 1;
                g.qr.v_len[qvs[t][i]] = pos + 1;
            }
    };
    // sum the four waves' partials in wave order (LDS reused after a barrier)
    __syncthreads();
    if (wave > 0) {
#pragma unroll
        for (int t = 0; t < RT; t++)
#pragma unroll
            for (int c = 0; c < CT; c++)
                *reinterpret_cast<f32x4_t*>(lds + (wave - 1) * kAcc + ((t * CT + c) * 64 + lane) * 16) = acc[t][c];
    }
    __syncthreads();
    if (wave == 0) {
#pragma unroll
        for (int w = 0; w < 3; w++)
#pragma unroll
            for (int t = 0; t < RT; t++)
#pragma unroll
                for (int c = 0; c < CT; c++)
                    acc[t][c] += *reinterpret_cast<const f32x4_t*>(lds + w * kAcc + ((t * CT + c) * 64 + lane) * 16);
    }

    const int64_t ob = bz * M * N;
    // q/k/v epilogue: each element's destination (null: none) and value,
    // stored together once every element is computed -- stores count in the
    // same counter as loads here, so a wait the compiler places between
    // address computations would otherwise wait for the earlier stores
    uint16_t* rp[ROPE ? RT : 1][ROPE ? CT : 1][4];
    uint16_t rv[ROPE ? RT : 1][ROPE ? CT : 1][4];
    auto rope_stores = [&]() {
#pragma unroll
        for (int t = 0; t < RT; t++)
#pragma unroll
            for (int c = 0; c < CT; c++)
#pragma unroll
                for (int i = 0; i < 4; i++)
                    if (rp[t][c][i]) *rp[t][c][i] = rv[t][c][i];
    };
    auto emit = [&](int t, int c, const f32x4_t& v) {
        const int64_t nc = n0 + 16 * c + (lane & 15);
        if constexpr (ROPE) {
            // the stored bf16 value of this lane's column and of its pair partner
            // (lane ^ 1), then the RoPE kernel's arithmetic: angle float(pos) /
            // denominator, rope_sincos, products and sum rounded separately,
            // bf16 round to nearest even
            // the argument fields read once per tile (inside the element loop the
            // compiler re-reads them with a scalar load and a wait per use)
            const int d = g.qr.d, hq = g.qr.hq, hkv = g.qr.hkv, shift = g.qr.page_shift;
            const int split_half = g.qr.split_half;
            const int32_t kmax = g.qr.k_max_blocks, vmax = g.qr.v_max_blocks;
            const int64_t page_bytes = g.qr.page_bytes;
            uint16_t* const q_out = g.qr.q_out;
            char* const k_pages = g.qr.k_pages;
            char* const v_pages = g.qr.v_pages;
            uint32_t* const errw = g.qr.errw;
            const int ncl = static_cast<int>(min<int64_t>(nc, N - 1));
            const int qk_cols = (hq + hkv) * d;
            const int head = static_cast<int>(static_cast<uint32_t>(ncl) / static_cast<uint32_t>(d));
            const int cp = ncl - head * d, pair = cp >> 1, second = ncl & 1;
            const int dst = split_half ? (second ? pair + (d >> 1) : pair) : cp;
            const int psz = 1 << shift;
            const float bias = g.bias ? bf16_to_f32(g.bias[ncl]) : 0.0f;
#pragma unroll
            for (int i = 0; i < 4; i++)
                asm volatile("" : "+v"(qpos[t][i]), "+v"(qkb[t][i]), "+v"(qvb[t][i]), "+v"(qkl[t][i]), "+v"(qvl[t][i]),
                             "+v"(qks[t][i]), "+v"(qvs[t][i]));
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int rr = static_cast<int>(r0) + 16 * t + 4 * (lane >> 4) + i;
                const float x = bf16_to_f32(f32_to_bf16(v[i] + bias));
                const float xp = lane_xor1(x);
                rp[t][c][i] = nullptr;
                if (rr >= M || nc >= N) continue;
                const int32_t pos = qpos[t][i];
                if (pos < 0) {
                    atomicOr(errw, static_cast<uint32_t>(SANDY_DEVERR_POSITION));
                    continue;
                }
                const int32_t bi = pos >> shift;
                const int32_t kb = bi < kmax ? qkb[t][i] : -1;
                const int32_t vb = bi < vmax ? qvb[t][i] : -1;
                // k and v are stored only where the row appends: at the sequence's
                // device length (a stale position would overwrite committed history)
                const bool at_len = qkl[t][i] == pos && qvl[t][i] == pos;
                const int row_in_page = pos & (psz - 1);
                if (ncl < qk_cols) {
                    const float x0 = second ? xp : x, x1 = second ? x : xp;
                    const float sn = qsn[t][i][c], cs = qcs[t][i][c];
                    rv[t][c][i] = second ? f32_to_bf16(__fadd_rn(__fmul_rn(x0, sn), __fmul_rn(x1, cs)))
                                         : f32_to_bf16(__fsub_rn(__fmul_rn(x0, cs), __fmul_rn(x1, sn)));
                    if (head < hq)
                        rp[t][c][i] = q_out + (rr * hq + head) * d + dst;
                    else if (kb >= 0 && at_len)
                        rp[t][c][i] = reinterpret_cast<uint16_t*>(k_pages + kb * page_bytes) +
                                      ((head - hq) * psz + row_in_page) * d + dst;
                } else {
                    rv[t][c][i] = f32_to_bf16(x);
                    if (vb >= 0 && at_len)
                        rp[t][c][i] = reinterpret_cast<uint16_t*>(v_pages + vb * page_bytes) +
                                      ((head - hq - hkv) * psz + row_in_page) * d + cp;
                }
                // the first k/v column tile, first column: the row's errors (the
                // lengths advance in rope_lengths)
                if (ct == kv_first && c == 0 && (lane & 15) == 0) {
                    if (kb < 0 || vb < 0) atomicOr(errw, static_cast<uint32_t>(SANDY_DEVERR_BLOCK));
                    if (!at_len) atomicOr(errw, static_cast<uint32_t>(SANDY_DEVERR_POSITION));
                }
            }
            return;
        }
        if (g.resid) {
            // out = bf16(resid + bf16(v)) (the GEMM's stored value, then the residual
            // add); the 16 lanes of a row reduce the squares of their 16 columns
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int64_t rr = r0 + 16 * t + 4 * (lane >> 4) + i;
                const bool in = nc < N && rr < M;
                const int64_t at = ob + (in ? rr * N + nc : 0);
                const uint16_t hv = static_cast<uint16_t>(rres[t][c][i >> 1] >> (16 * (i & 1)));
                const float sv = bf16_to_f32(f32_to_bf16(__fadd_rn(bf16_to_f32(f32_to_bf16(v[i])), bf16_to_f32(hv))));
                if (in) g.out[at] = f32_to_bf16(sv);
                const double sq = group_sum<16>(in ? static_cast<double>(sv) * static_cast<double>(sv) : 0.0);
                if ((lane & 15) == 0 && rr < M && g.rsq_out)
                    g.rsq_out[(bz * M + rr) * g.rsq_parts + (n0 >> 4) + c] = sq;
            }
            return;
        }
        if (g.glu) {
            // columns (2i, 2i + 1) = (gate_i, up_i) sit in lanes (l, l ^ 1); both
            // are rounded to bf16 as the plain GEMM would store them, and the
            // even lane writes act[row, i] of the [M, N / 2] output (every lane
            // takes part in the shuffle)
            const int64_t half = N >> 1;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float gv = bf16_to_f32(f32_to_bf16(v[i]));
                const float uv = lane_xor1(gv);
                const int64_t rr = r0 + 16 * t + 4 * (lane >> 4) + i;
                if ((lane & 1) == 0 && nc < N && rr < M)
                    g.out[(bz * M + rr) * half + (nc >> 1)] = f32_to_bf16(glu_pair(g.glu, gv, uv));
            }
            return;
        }
        if (nc >= N) return;
        const float bias = g.bias ? bf16_to_f32(g.bias[nc]) : 0.0f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int64_t rr = r0 + 16 * t + 4 * (lane >> 4) + i;
            if (rr < M) g.out[ob + rr * N + nc] = f32_to_bf16(v[i] + bias);
        }
    };
    if (g.splits == 1) {
        if (wave == 0)
#pragma unroll
            for (int t = 0; t < RT; t++)
#pragma unroll
                for (int c = 0; c < CT; c++) emit(t, c, acc[t][c]);
        if constexpr (ROPE)
            if (wave == 0) {
                rope_stores();
                rope_lengths();
            }
        return;
    }
    // split-K across workgroups: partials written through to the agent's coherence
    // point, then the last-arriving workgroup of the tile sums them (wave 0 holds the tile)
    const int64_t tile = (bz * g.row_tiles + blockIdx.y) * g.col_tiles + ct;
    constexpr int kTileFloats = RT * CT * 64 * 4;
    float* pbase = g.part + tile * g.splits * kTileFloats;
    if (wave == 0) {
#pragma unroll
        for (int t = 0; t < RT; t++)
#pragma unroll
            for (int c = 0; c < CT; c++) {
                uint64_t* p = reinterpret_cast<uint64_t*>(pbase + split * kTileFloats + ((t * CT + c) * 64 + lane) * 4);
                __hip_atomic_store(p, static_cast<uint64_t>(__float_as_uint(acc[t][c][0])) |
                                          (static_cast<uint64_t>(__float_as_uint(acc[t][c][1])) << 32),
                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_store(p + 1, static_cast<uint64_t>(__float_as_uint(acc[t][c][2])) |
                                              (static_cast<uint64_t>(__float_as_uint(acc[t][c][3])) << 32),
                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
    }
    __shared__ int is_last;
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid == 0) {
        uint32_t* ctr = g.counters + tile;
        const uint32_t prev = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        is_last = prev == static_cast<uint32_t>(g.splits - 1);
        if (is_last) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if constexpr (ROPE)
        if (wave == 0 && !is_last) rope_lengths();
    if (!is_last || wave != 0) return;
#pragma unroll
    for (int t = 0; t < RT; t++)
#pragma unroll
        for (int c = 0; c < CT; c++) {
            f32x4_t sum = f32x4_t{0.f, 0.f, 0.f, 0.f};
            const int64_t off = ((t * CT + c) * 64 + lane) * 4;
            for (int s0 = 0; s0 < g.splits; s0 += 8) {
                uint64_t w0[8], w1[8];
#pragma unroll
                for (int q = 0; q < 8; q++) {
                    const int s = s0 + q < g.splits ? s0 + q : s0;
                    uint64_t* p = reinterpret_cast<uint64_t*>(pbase + s * kTileFloats + off);
                    w0[q] = __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    w1[q] = __hip_atomic_load(p + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
#pragma unroll
                for (int q = 0; q < 8; q++) {
                    if (s0 + q >= g.splits) break;
                    sum[0] += __uint_as_float(static_cast<uint32_t>(w0[q]));
                    sum[1] += __uint_as_float(static_cast<uint32_t>(w0[q] >> 32));
                    sum[2] += __uint_as_float(static_cast<uint32_t>(w1[q]));
                    sum[3] += __uint_as_float(static_cast<uint32_t>(w1[q] >> 32));
                }
            }
            emit(t, c, sum);
        }
    if constexpr (ROPE) {
        rope_stores();
        rope_lengths();
    }
}


// Launchers of gemm_waves_kernel, one translation unit per (form, NT) so they
// compile in parallel: tile variant as in the host heuristic of matmul.hip
// ((RT, CT) = 0 (1, 1), 1 (2, 1), 3 (2, 2), 4 (1, 2), 5 (2, 4), 6 (1, 4)), run
// length cps, chunks in flight qdepth.
// plain (matmul_waves.hip, matmul_waves_nt.hip)
template <bool NT>
void launch_waves_plain(int variant, int cps, int qdepth, dim3 grid, hipStream_t stream, const GemmArgs& g);
// with the RMSNorm prologue (matmul_norm.hip, matmul_norm_nt.hip)
template <bool NT>
void launch_waves_norm(int variant, int cps, int qdepth, dim3 grid, hipStream_t stream, const GemmArgs& g);
// with the q/k/v epilogue (matmul_qkv.hip, matmul_qkv_nt.hip): RT 1, CT 1 or 2
// (variant 0 or 4), four chunks in flight from run length 4
template <bool NT>
void launch_waves_qkv(int variant, int cps, int qdepth, bool norm, dim3 grid, hipStream_t stream, const GemmArgs& g);
extern template void launch_waves_plain<false>(int, int, int, dim3, hipStream_t, const GemmArgs&);
extern template void launch_waves_plain<true>(int, int, int, dim3, hipStream_t, const GemmArgs&);
extern template void launch_waves_norm<false>(int, int, int, dim3, hipStream_t, const GemmArgs&);
extern template void launch_waves_norm<true>(int, int, int, dim3, hipStream_t, const GemmArgs&);
extern template void launch_waves_qkv<false>(int, int, int, bool, dim3, hipStream_t, const GemmArgs&);
extern template void launch_waves_qkv<true>(int, int, int, bool, dim3, hipStream_t, const GemmArgs&);

// The q/k/v decode GEMM with the RoPE + paged-append epilogue (QkvRope
// filled in by the caller except its pointers' validation): lhs [m, k] bf16,
// rhs [n, k] bf16 with n = (hq + 2 hkv) d; with lhs_stats and norm_weight the
// RMSNorm prologue of sandy_hip_matmul_rms.  dry: run every check and take
// the workspace, launch nothing (so a caller can validate before it moves
// bookkeeping).  Defined in matmul.hip.
int matmul_qkv(const SandyTensor* lhs, const SandyRowStats* lhs_stats, const SandyTensor* norm_weight, double eps,
               const SandyTensor* rhs, const QkvRope& qr, hipStream_t stream, Err e, bool dry = false);

} // namespace sandy_hip
