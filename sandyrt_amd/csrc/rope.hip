// rope.hip -- rotary position embedding (RoPEKernelOp).
//
// Semantics: src/core/TensorCalc.cpp:1823-1937 (rope_impl).  Vector v of the
// input ([..., seq, dim]) sits at position v % seq, or takes it from
// position_ids (numel 1: ids[0] + v % seq; numel == vectors: ids[v];
// numel == seq: ids[v % seq]).  Split-half rotates (x[i], x[i + dim/2]) by
// pos / theta^(2i / dim); interleaved rotates (x[2i], x[2i+1]) by
// pos / theta^(2i / rotary_dim); pairs past rotary_dim/2 are copied.
//
// The denominators theta^(2i/d) are evaluated on the host with the same
// powf the CPU reference uses and passed as kernel arguments, so every angle
// (a correctly rounded division on gfx950) equals the CPU's bit for bit; only
// cos/sin differ, within an ulp (evaluation below).  The reference CUDA kernel
// evaluates powf per pair on the device and synchronises the host after every
// launch to read an error flag (CudaRoPEKernels.cu:272-333); here a negative
// position sets the sticky device error word instead.
//
// gfx950 design: when positions depend only on the sequence index, one thread
// owns (sequence position, 8 pairs, a group of heads): it issues the loads of
// up to four heads first (2 x 16 B each, 128-bit), evaluates its 8 sin/cos
// pairs while they are in flight, and reuses them for every head of its
// group.  C2's q [1, 32, 4096, 64] therefore spends 1/4 of a sin/cos per
// element and stays HBM-bound.
//
// sin/cos: the angle (a float, bit-identical to the CPU's) is reduced by
// Cody-Waite in double precision, r = a - k * pi/2 with pi/2 split in two
// doubles (exact for the |a| < 2^20 that positions reach), then sin and cos
// of |r| <= pi/4 are Taylor polynomials to r^11 / r^12 in float and the
// quadrant k mod 4 selects and signs them.  Within 1 ulp of a correctly
// rounded result, like the CPU's sinf/cosf, at a fraction of the cost of the
// device libm's sincosf for large arguments (which made this kernel
// compute-bound: 9.2 vs 7.8 us for C2's q).
#include "common.h"

#include <cmath>
#include <cstdlib>

namespace sandy_hip {
namespace {

constexpr int kMaxPairs = 256;  // rotary dims up to 512

struct RopeArgs {
    float denom[kMaxPairs];
};

// mode: 0 = position from sequence index, 1 = ids[0] + seq index,
//       2 = ids[seq index], 3 = ids[vector]
__device__ __forceinline__ int64_t rope_position(int mode, const void* ids, int32_t ids_dt, int64_t vec, int64_t s,
                                                 uint32_t* errw) {
    int64_t p = s;
    if (mode == 1) p = load_index(ids, ids_dt, 0) + s;
    else if (mode == 2) p = load_index(ids, ids_dt, s);
    else if (mode == 3) p = load_index(ids, ids_dt, vec);
    if (p < 0) {
        atomicOr(errw, static_cast<uint32_t>(SANDY_DEVERR_POSITION));
        p = 0;
    }
    return p;
}

// The position of mode/vec/s in two steps: rope_position_words requests the
// raw words from a branch-free address (a valid dummy word when the mode needs
// none) and rope_position_join assembles and range-checks them at the first
// use, so the loads issued in between are not waited for behind it (a branch
// on the loaded value, or the sign extension of an int32 id, is a use).
struct RopeWords {
    uint32_t lo, hi;
};

__device__ __forceinline__ RopeWords rope_position_words(int mode, const void* ids, int32_t ids_dt, int64_t vec,
                                                         int64_t s, const uint32_t* dummy) {
    const bool i32 = ids_dt == SANDY_I32;
    const int64_t idx = mode == 2 ? s : mode == 3 ? vec : 0;
    const uint32_t* p = mode == 0 ? dummy : static_cast<const uint32_t*>(ids) + (i32 ? idx : 2 * idx);
    RopeWords w;
    w.lo = p[0];
    w.hi = p[i32 || mode == 0 ? 0 : 1];
    return w;
}

__device__ __forceinline__ int64_t rope_position_join(int mode, int32_t ids_dt, RopeWords w, int64_t s) {
    if (mode == 0) return s;
    const int64_t v = ids_dt == SANDY_I32 ? static_cast<int64_t>(static_cast<int32_t>(w.lo))
                                          : static_cast<int64_t>((static_cast<uint64_t>(w.hi) << 32) | w.lo);
    return mode == 1 ? v + s : v;
}

// Split-half, 8 pairs per thread, loads of U heads issued before the sin/cos.
// grid: (seq * chunks * groups) threads.  FULL: every group holds a multiple
// of U heads and every pair rotates, so no guards (the per-load and per-pair
// branches cost 15% of the kernel's time).
template <typename T, int U, bool FULL>
__global__ __launch_bounds__(256) void rope_split_kernel(
        const void* __restrict__ x, void* __restrict__ out, const void* __restrict__ x2, void* __restrict__ out2,
        int64_t outer_first, const void* __restrict__ ids, int32_t ids_dt, int mode, int64_t seq, int64_t outer,
        int dim, int rot_pairs, int groups, int per_group, RopeArgs args, uint32_t* errw) {
    const int half = dim >> 1;
    const uint32_t chunks = static_cast<uint32_t>(half >> 3);
    // 32-bit index math (the host keeps seq * chunks * groups below 2^31):
    // 64-bit divisions by runtime values delayed the first load measurably
    const uint32_t t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= static_cast<uint32_t>(seq) * chunks * static_cast<uint32_t>(groups)) return;
    const int c = static_cast<int>(t % chunks);
    const uint32_t rest = t / chunks;
    const int64_t s = rest % static_cast<uint32_t>(seq);
    const int g = static_cast<int>(rest / static_cast<uint32_t>(seq));
    const int64_t o_begin = static_cast<int64_t>(g) * per_group;
    const int64_t o_end = min(outer, o_begin + per_group);
    float cs[8], sn[8];
    int64_t pos = -1;
    for (int64_t o0 = o_begin; o0 < o_end; o0 += U) {
        // the position (possibly a load of position_ids) is read before the
        // data loads: memory-load counters retire in order, so waiting for a
        // later small load would also wait for every data load before it
        const bool fresh = mode == 3 || pos < 0;  // mode 3 runs with one head per group
        if (fresh) pos = rope_position(mode, ids, ids_dt, o0 * seq + s, s, errw);
        typename Vec8<T>::raw ra_[U], rb_[U];
#pragma unroll
        for (int j = 0; j < U; j++) {
            if (FULL || o0 + j < o_end) {
                const bool sec = o0 + j >= outer_first;
                const int64_t base = ((o0 + j - (sec ? outer_first : 0)) * seq + s) * dim;
                ra_[j] = Vec8<T>::load_raw(sec ? x2 : x, base + c * 8);
                rb_[j] = Vec8<T>::load_raw(sec ? x2 : x, base + half + c * 8);
            }
        }
        if (fresh) {
            const float fp = static_cast<float>(pos);
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const int p = c * 8 + i;
                if (FULL || p < rot_pairs) rope_sincos(fp / args.denom[p], &sn[i], &cs[i]);
            }
        }
#pragma unroll
        for (int j = 0; j < U; j++) {
            if (!FULL && o0 + j >= o_end) break;
            const bool sec = o0 + j >= outer_first;
            const int64_t base = ((o0 + j - (sec ? outer_first : 0)) * seq + s) * dim;
            void* dst = sec ? out2 : out;
            float a[8], b[8], ra[8], rb[8];
            Vec8<T>::unpack(ra_[j], a);
            Vec8<T>::unpack(rb_[j], b);
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const int p = c * 8 + i;
                if (FULL || p < rot_pairs) {
                    ra[i] = __fsub_rn(__fmul_rn(a[i], cs[i]), __fmul_rn(b[i], sn[i]));
                    rb[i] = __fadd_rn(__fmul_rn(a[i], sn[i]), __fmul_rn(b[i], cs[i]));
                } else {
                    ra[i] = a[i];
                    rb[i] = b[i];
                }
            }
            Vec8<T>::store(dst, base + c * 8, ra);
            Vec8<T>::store(dst, base + half + c * 8, rb);
        }
    }
}

// Split-half rotation with whole-line accesses: the 2 * chunks lanes of a
// row (a power of two dividing 64) each load and store one 16- or 32-byte
// piece, the first chunks lanes from the first half and the rest from the
// second, so every load and store instruction covers whole rows instead of
// one half of each.  Each lane takes its partner's piece (the same piece
// index in the other half) by a lane exchange, and computes the sin/cos of four of its eight pairs, taking
// the other four from its partner.  Same arithmetic as
// rope_split_kernel.
// TAB: the cos/sin of every (sequence index, pair) come from a table built
// by rope_cache_kernel (one [seq, rot_pairs] float2 table shared by q, k and
// every layer of a forward pass) instead of being evaluated here.
// XCH: how a lane reaches its partner.  0: ds_bpermute to lane ^ chunks;
// otherwise a DPP mirror (0x141 row_half_mirror for 8 lanes a row, 0x140
// row_mirror for 16) with the second half's pieces laid out in reverse lane
// order, so the mirrored lane holds the partner piece (one VALU move per word
// instead of an LDS-crossbar round trip: 8.52-8.60 -> 8.45-8.47 us at config 2).
template <typename T, int U, bool FULL, bool TAB = false, int XCH = 0>
__global__ __launch_bounds__(256) void rope_split_lines_kernel(
        const void* __restrict__ x, void* __restrict__ out, const void* __restrict__ x2, void* __restrict__ out2,
        int64_t outer_first, const void* __restrict__ ids, int32_t ids_dt, int mode, int64_t seq, int64_t outer,
        int dim, int rot_pairs, int groups, int per_group, RopeArgs args, uint32_t* errw,
        const float2* __restrict__ tab = nullptr) {
    const int half = dim >> 1;
    const uint32_t chunks = static_cast<uint32_t>(half >> 3);
    const uint32_t lanes = 2 * chunks;
    const uint32_t t = blockIdx.x * blockDim.x + threadIdx.x;
    // row-granular exit: a row's lanes leave together, partners stay paired
    if (t >= static_cast<uint32_t>(seq) * lanes * static_cast<uint32_t>(groups)) return;
    const uint32_t r = t & (lanes - 1);
    const bool hi = r >= chunks;
    const int c = static_cast<int>(XCH != 0 && hi ? lanes - 1 - r : r & (chunks - 1));
    const uint32_t rest = t / lanes;
    const int64_t s = rest % static_cast<uint32_t>(seq);
    const int g = static_cast<int>(rest / static_cast<uint32_t>(seq));
    const int64_t o_begin = static_cast<int64_t>(g) * per_group;
    const int64_t o_end = min(outer, o_begin + per_group);
    const int m = static_cast<int>(chunks);
    auto partner = [&](uint32_t v) -> uint32_t {
        if constexpr (XCH != 0) return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), XCH, 0xf, 0xf, false));
        else return static_cast<uint32_t>(__shfl_xor(static_cast<int>(v), m, 64));
    };
    float cs[8], sn[8];
    bool have = false;
    for (int64_t o0 = o_begin; o0 < o_end; o0 += U) {
        const bool fresh = mode == 3 || !have;
        // issue order: the position and this lane's angle denominators (their
        // waits then leave the rows in flight), the cos/sin table entries, the
        // rows; the position is range-checked once the rows are requested
        RopeWords pw{0, 0};
        float den4[4];
        if (!TAB && fresh) {
            // mode 0 needs no position word: the sin/cos then depend on no
            // vector load and are computed while the rows are in flight
            if (mode != 0) pw = rope_position_words(mode, ids, ids_dt, o0 * seq + s, s, errw);
            if (chunks <= 4) {
                // rows of up to 64 pairs: every candidate denominator is a
                // uniform (scalar) load, selected by the lane's quarter-chunk
                // (constant offsets into the argument block: the first 32
                // denominators in scalar registers; entries past rot_pairs
                // feed only pairs that pass through unrotated)
                // (readfirstlane keeps each value a scalar: a select between
                // loads would otherwise become one per-lane vector load)
                const int sel = 2 * c + (hi ? 1 : 0);
                int all[32];
#pragma unroll
                for (int q = 0; q < 32; q++) all[q] = __builtin_amdgcn_readfirstlane(__float_as_int(args.denom[q]));
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    int d = all[i];
#pragma unroll
                    for (int q = 1; q < 8; q++) d = q == sel ? all[4 * q + i] : d;
                    den4[i] = __int_as_float(d);
                }
            } else {
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int p = c * 8 + (hi ? 4 : 0) + i;
                    den4[i] = args.denom[FULL || p < rot_pairs ? p : 0];
                }
            }
        }
        float2 tv[4];
        if (TAB && fresh) {  // requested with the row's loads
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int p = c * 8 + (hi ? 4 : 0) + i;
                tv[i] = tab[s * rot_pairs + (FULL || p < rot_pairs ? p : 0)];
            }
        }
        typename Vec8<T>::raw mine[U];
#pragma unroll
        for (int j = 0; j < U; j++) {
            if (FULL || o0 + j < o_end) {
                const bool sec = o0 + j >= outer_first;
                const int64_t base = ((o0 + j - (sec ? outer_first : 0)) * seq + s) * dim;
                mine[j] = Vec8<T>::load_raw_nt(sec ? x2 : x, base + (hi ? half : 0) + c * 8);
            }
        }
        if (fresh) {
            int64_t pos = TAB ? 0 : rope_position_join(mode, ids_dt, pw, s);
            if (pos < 0) {
                atomicOr(errw, static_cast<uint32_t>(SANDY_DEVERR_POSITION));
                pos = 0;
            }
            have = true;
            const float fp = static_cast<float>(pos);
            float s4[4], c4[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int p = c * 8 + (hi ? 4 : 0) + i;
                s4[i] = 0.0f;
                c4[i] = 1.0f;
                if (TAB) {
                    if (FULL || p < rot_pairs) {
                        c4[i] = tv[i].x;
                        s4[i] = tv[i].y;
                    }
                } else if (FULL || p < rot_pairs) {
                    rope_sincos(fp / den4[i], &s4[i], &c4[i]);
                }
            }
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float so = __uint_as_float(partner(__float_as_uint(s4[i])));
                const float co = __uint_as_float(partner(__float_as_uint(c4[i])));
                sn[i] = hi ? so : s4[i];
                cs[i] = hi ? co : c4[i];
                sn[4 + i] = hi ? s4[i] : so;
                cs[4 + i] = hi ? c4[i] : co;
            }
        }
#pragma unroll
        for (int j = 0; j < U; j++) {
            // every lane of a row takes the same branch here (o_end is per row group)
            if (!FULL && o0 + j >= o_end) break;
            // the partner lane's piece by a lane exchange: the rows are read
            // once, non-temporal (8.8 -> 8.5 us at config 2 against re-reading the
            // partner's piece from the cached line: 8.8-8.9 with plain loads,
            // 9.3-9.7 with non-temporal ones; ds_swizzle 9.1-9.3)
            typename Vec8<T>::raw other;
            {
                const uint32_t* src = reinterpret_cast<const uint32_t*>(&mine[j]);
                uint32_t* dst = reinterpret_cast<uint32_t*>(&other);
#pragma unroll
                for (int w = 0; w < static_cast<int>(sizeof(mine[j]) / 4); w++) dst[w] = partner(src[w]);
            }
            const bool sec = o0 + j >= outer_first;
            const int64_t base = ((o0 + j - (sec ? outer_first : 0)) * seq + s) * dim;
            float a[8], b[8], res[8];
            Vec8<T>::unpack(hi ? other : mine[j], a);
            Vec8<T>::unpack(hi ? mine[j] : other, b);
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const int p = c * 8 + i;
                if (FULL || p < rot_pairs)
                    res[i] = hi ? __fadd_rn(__fmul_rn(a[i], sn[i]), __fmul_rn(b[i], cs[i]))
                                : __fsub_rn(__fmul_rn(a[i], cs[i]), __fmul_rn(b[i], sn[i]));
                else
                    res[i] = hi ? b[i] : a[i];
            }
            Vec8<T>::store(sec ? out2 : out, base + (hi ? half : 0) + c * 8, res);
        }
    }
}

// Interleaved, 4 pairs (8 elements) per thread, loads of U heads first;
// FULL as for the split-half kernel.
template <typename T, int U, bool FULL>
__global__ __launch_bounds__(256) void rope_interleaved_kernel(
        const void* __restrict__ x, void* __restrict__ out, const void* __restrict__ x2, void* __restrict__ out2,
        int64_t outer_first, const void* __restrict__ ids, int32_t ids_dt, int mode, int64_t seq, int64_t outer,
        int dim, int rot_pairs, int groups, int per_group, RopeArgs args, uint32_t* errw) {
    const uint32_t chunks = static_cast<uint32_t>(dim >> 3);
    const uint32_t t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= static_cast<uint32_t>(seq) * chunks * static_cast<uint32_t>(groups)) return;
    const int c = static_cast<int>(t % chunks);
    const uint32_t rest = t / chunks;
    const int64_t s = rest % static_cast<uint32_t>(seq);
    const int g = static_cast<int>(rest / static_cast<uint32_t>(seq));
    const int64_t o_begin = static_cast<int64_t>(g) * per_group;
    const int64_t o_end = min(outer, o_begin + per_group);
    float cs[4], sn[4];
    int64_t pos = -1;
    for (int64_t o0 = o_begin; o0 < o_end; o0 += U) {
        const bool fresh = mode == 3 || pos < 0;  // position before the data loads, as above
        if (fresh) pos = rope_position(mode, ids, ids_dt, o0 * seq + s, s, errw);
        typename Vec8<T>::raw raw_[U];
#pragma unroll
        for (int j = 0; j < U; j++)
            if (FULL || o0 + j < o_end) {
                const bool sec = o0 + j >= outer_first;
                raw_[j] = Vec8<T>::load_raw(sec ? x2 : x, ((o0 + j - (sec ? outer_first : 0)) * seq + s) * dim + c * 8);
            }
        if (fresh) {
            const float fp = static_cast<float>(pos);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int p = c * 4 + i;
                if (FULL || p < rot_pairs) rope_sincos(fp / args.denom[p], &sn[i], &cs[i]);
            }
        }
#pragma unroll
        for (int j = 0; j < U; j++) {
            if (!FULL && o0 + j >= o_end) break;
            float a[8], r[8];
            Vec8<T>::unpack(raw_[j], a);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int p = c * 4 + i;
                if (FULL || p < rot_pairs) {
                    r[2 * i] = __fsub_rn(__fmul_rn(a[2 * i], cs[i]), __fmul_rn(a[2 * i + 1], sn[i]));
                    r[2 * i + 1] = __fadd_rn(__fmul_rn(a[2 * i], sn[i]), __fmul_rn(a[2 * i + 1], cs[i]));
                } else {
                    r[2 * i] = a[2 * i];
                    r[2 * i + 1] = a[2 * i + 1];
                }
            }
            const bool sec = o0 + j >= outer_first;
            Vec8<T>::store(sec ? out2 : out, ((o0 + j - (sec ? outer_first : 0)) * seq + s) * dim + c * 8, r);
        }
    }
}

// Generic: one thread per pair, strided tensors, any dims.
struct Strided {
    int64_t dims[SANDY_HIP_MAX_RANK];
    int64_t xs[SANDY_HIP_MAX_RANK];
    int64_t os[SANDY_HIP_MAX_RANK];
    int rank;
};

__device__ __forceinline__ void offsets(const Strided& st, int64_t linear, int64_t& xo, int64_t& oo) {
    xo = 0;
    oo = 0;
    for (int d = st.rank - 1; d >= 0; d--) {
        const int64_t c = linear % st.dims[d];
        linear /= st.dims[d];
        xo += c * st.xs[d];
        oo += c * st.os[d];
    }
}

__global__ __launch_bounds__(256) void rope_generic_kernel(
        const void* __restrict__ x, int32_t dt, void* __restrict__ out, const void* __restrict__ ids, int32_t ids_dt,
        int mode, int64_t seq, int64_t vectors, int dim, int rot_pairs, int split, Strided st, RopeArgs args,
        uint32_t* errw) {
    const int pairs = dim >> 1;
    const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (t >= vectors * pairs) return;
    const int p = static_cast<int>(t % pairs);
    const int64_t vec = t / pairs;
    const int64_t s = vec % seq;
    const int64_t i0 = split ? p : 2 * p;
    const int64_t i1 = split ? p + pairs : 2 * p + 1;
    int64_t x0, o0, x1, o1;
    offsets(st, vec * dim + i0, x0, o0);
    offsets(st, vec * dim + i1, x1, o1);
    const float a = load_any(x, dt, x0);
    const float b = load_any(x, dt, x1);
    if (p >= rot_pairs) {
        store_any(out, dt, o0, a);
        store_any(out, dt, o1, b);
        return;
    }
    const int64_t pos = rope_position(mode, ids, ids_dt, vec, s, errw);
    float sn, cs;
    rope_sincos(static_cast<float>(pos) / args.denom[p], &sn, &cs);
    store_any(out, dt, o0, __fsub_rn(__fmul_rn(a, cs), __fmul_rn(b, sn)));
    store_any(out, dt, o1, __fadd_rn(__fmul_rn(a, sn), __fmul_rn(b, cs)));
}

// The cos/sin table: entry (s, p) = (cos, sin) of position(s) / denom[p],
// the same float angle and rope_sincos as the kernels above.
__global__ __launch_bounds__(256) void rope_cache_kernel(const void* __restrict__ ids, int32_t ids_dt, int mode,
                                                         int64_t seq, int rot_pairs, RopeArgs args, uint32_t* errw,
                                                         float2* __restrict__ tab) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (t >= seq * rot_pairs) return;
    const int64_t s = t / rot_pairs;
    const int p = static_cast<int>(t - s * rot_pairs);
    const int64_t pos = rope_position(mode, ids, ids_dt, s, s, errw);
    float sn, cs;
    rope_sincos(static_cast<float>(pos) / args.denom[p], &sn, &cs);
    tab[t] = make_float2(cs, sn);
}

} // namespace
} // namespace sandy_hip

using namespace sandy_hip;

namespace sandy_hip {
namespace {

struct RopeShape {
    int64_t seq, dim, total, vectors, outer;
};

// Validation shared by both entry points; fills the shape of x.
int rope_check(const SandyTensor* x, const SandyTensor* out, RopeShape& sh, Err e) {
    if (!valid_rank(x) || !valid_rank(out)) return fail(e, SANDY_ERR_INVALID, "rope tensor rank out of range");
    if (!is_float(x->dtype)) return fail(e, SANDY_ERR_INVALID, "rope input unsupported dtype");
    if (!same_shape(*x, *out)) return fail(e, SANDY_ERR_INVALID, "rope output shape mismatch");
    if (out->dtype != x->dtype) return fail(e, SANDY_ERR_INVALID, "rope output dtype mismatch");
    if (x->rank < 2) return fail(e, SANDY_ERR_INVALID, "rope input must have rank >= 2");
    sh.seq = x->dims[x->rank - 2];
    sh.dim = x->dims[x->rank - 1];
    if (sh.dim <= 0 || sh.dim % 2 != 0) return fail(e, SANDY_ERR_INVALID, "rope last dimension must be positive and even");
    sh.total = numel(*x);
    sh.vectors = sh.total / sh.dim;
    sh.outer = sh.seq ? sh.vectors / sh.seq : 0;
    return SANDY_OK;
}

// RoPE of n = 1 or 2 tensors sharing the positions, sequence length and head
// dim (checked by the caller); the fast kernels take both in one launch.
int rope_run(const SandyTensor* const* xs, const SandyTensor* const* outs, int n, const SandyTensor* position_ids,
             double theta, int64_t rotary_dim, int32_t split_half, hipStream_t stream, Err e) {
    RopeShape sh[2];
    for (int i = 0; i < n; i++) {
        const int st = rope_check(xs[i], outs[i], sh[i], e);
        if (st) return st;
    }
    if (position_ids && !is_index(position_ids->dtype))
        return fail(e, SANDY_ERR_INVALID, "rope position_ids must be i32 or i64");
    const float th = static_cast<float>(theta);
    if (th <= 0.0f) return fail(e, SANDY_ERR_INVALID, "rope theta must be > 0");
    const int64_t seq = sh[0].seq, dim = sh[0].dim;
    if (rotary_dim < 0) rotary_dim = dim;
    if (rotary_dim <= 0 || rotary_dim % 2 != 0) return fail(e, SANDY_ERR_INVALID, "rope rotary_dim must be positive and even");
    if (rotary_dim > dim) return fail(e, SANDY_ERR_INVALID, "rope rotary_dim must be <= last dimension");
    if (rotary_dim / 2 > kMaxPairs) return fail(e, SANDY_ERR_UNSUPPORTED, "rope rotary_dim above %d", 2 * kMaxPairs);
    int mode[2] = {0, 0};
    for (int i = 0; i < n; i++) {
        if (!position_ids) continue;
        const int64_t cnt = numel(*position_ids);
        if (cnt != 1 && cnt != seq && cnt != sh[i].vectors)
            return fail(e, SANDY_ERR_INVALID, "rope position_ids numel must be 1, sequence length, or vector count");
        if (!contiguous(*position_ids)) return fail(e, SANDY_ERR_UNSUPPORTED, "rope position_ids must be contiguous");
        mode[i] = cnt == 1 ? 1 : (cnt == sh[i].vectors && cnt != seq ? 3 : 2);
        if (mode[i] == 3 && sh[i].outer == 1) mode[i] = 2;  // ids[v] == ids[v % seq] when there is one sequence
    }
    RopeArgs args{};
    const int rot_pairs = static_cast<int>(rotary_dim / 2);
    const float div = static_cast<float>(split_half ? dim : rotary_dim);
    for (int p = 0; p < rot_pairs; p++) args.denom[p] = std::pow(th, static_cast<float>(2 * p) / div);
    int status = 0;
    uint32_t* errw = device_error_word(e, &status);
    if (status) return status;
    const void* ids = position_ids ? base_ptr(*position_ids) : nullptr;
    const int32_t ids_dt = position_ids ? position_ids->dtype : SANDY_I64;
    const bool bf = xs[0]->dtype == SANDY_BF16;
    // one launch over both tensors' heads when both take the fast kernels with
    // one position rule (per-vector ids differ between the tensors)
    bool fast = n == 1 || (mode[0] == mode[1] && mode[0] != 3);
    int64_t total = 0, outer = 0;
    for (int i = 0; i < n; i++) {
        const void* px = base_ptr(*xs[i]);
        const void* po = base_ptr(*outs[i]);
        const bool aligned = ((reinterpret_cast<uintptr_t>(px) | reinterpret_cast<uintptr_t>(po)) & 15u) == 0;
        fast = fast && contiguous(*xs[i]) && contiguous(*outs[i]) && aligned &&
               (split_half ? (dim / 2) % 8 == 0 : dim % 8 == 0);
        total += sh[i].total;
        outer += sh[i].outer;
    }
    if (total == 0) return ok(e);
    int groups = 1, per = 1;
    int64_t threads = 0;
    bool lines = false;
    if (fast) {
        const int chunks = static_cast<int>(split_half ? dim / 16 : dim / 8);
        // split-half rows whose two halves fit one shuffle group take the
        // whole-line kernel (twice the lanes, each with one piece)
        lines = split_half && chunks <= 32 && (chunks & (chunks - 1)) == 0;
        const int64_t base_threads = seq * chunks * (lines ? 2 : 1);
        if (mode[0] == 3) {
            groups = static_cast<int>(outer);
        } else {
            // threads (each reusing its sincos over `per` heads): numel / 32 within
            // [32K, 128K] -- measured best for C2's q (128K) and k (32K) on gfx950
            const int64_t want = std::min<int64_t>(131072, std::max<int64_t>(32768, total / 32));
            // (counted in pieces of 16 elements per row for either kernel)
            const int64_t row_threads = seq * chunks;
            groups = static_cast<int>(std::min<int64_t>(outer, std::max<int64_t>(1, want / std::max<int64_t>(1, row_threads))));
            per = static_cast<int>((outer + groups - 1) / groups);
            // prefer a head count per group that divides the heads (unguarded kernel)
            for (int d = per; d > 1 && d * 2 > per; d--)
                if (outer % d == 0) {
                    per = d;
                    break;
                }
            groups = static_cast<int>((outer + per - 1) / per);
            // the whole-line kernel: 6 heads per group (one batch of loads, the
            // sin/cos shared by 6 heads) when the heads divide by 6 and at
            // least 96K threads remain (config 2's 36 heads: 9.4 -> 9.2 us)
            if (lines && per < 6 && outer % 6 == 0 && 2 * row_threads * (outer / 6) >= 98304) {
                per = 6;
                groups = static_cast<int>(outer / 6);
            }
        }
        threads = base_threads * groups;
        if (threads + 255 >= (int64_t(1) << 31)) fast = false;  // the fast kernels index threads in 32 bits
    }
    if (fast) {
        dim3 grid(static_cast<unsigned>((threads + 255) / 256));
        const void* px = base_ptr(*xs[0]);
        void* po = base_ptr(*outs[0]);
        const void* px2 = n == 2 ? base_ptr(*xs[1]) : px;
        void* po2 = n == 2 ? base_ptr(*outs[1]) : po;
        const int64_t outer_first = sh[0].outer;
        const int md = mode[0];
        // up to four heads' loads in flight per thread (mode 3 has one head per group)
        int u = per >= 4 ? 4 : (per >= 2 ? 2 : 1);
        if (lines && per == 6) u = 6;  // the whole-line kernel takes 6 heads' loads at once
        const bool full = outer % per == 0 && per % u == 0 && rot_pairs == dim / 2;
#define SANDY_ROPE_LAUNCH(KERNEL, T, U, F, ...)                                                                   \
    hipLaunchKernelGGL((KERNEL<T, U, F, ##__VA_ARGS__>), grid, dim3(256), 0, stream, px, po, px2, po2, outer_first, ids, ids_dt, \
                       md, seq, outer, static_cast<int>(dim), rot_pairs, groups, per, args, errw)
#define SANDY_ROPE_F(KERNEL, T, U)                                 \
    do {                                                           \
        if (full) SANDY_ROPE_LAUNCH(KERNEL, T, U, true);           \
        else SANDY_ROPE_LAUNCH(KERNEL, T, U, false);               \
    } while (0)
#define SANDY_ROPE_U(KERNEL, T)                         \
    do {                                                \
        if (u == 4) SANDY_ROPE_F(KERNEL, T, 4);         \
        else if (u == 2) SANDY_ROPE_F(KERNEL, T, 2);    \
        else SANDY_ROPE_F(KERNEL, T, 1);                \
    } while (0)
        if (lines) {
            // the partner exchange by DPP mirror for 8 or 16 lanes a row (half = 32 or 64 elements)
            const int lane_count = static_cast<int>(dim / 8);
#define SANDY_ROPE_LINES(T, U, F)                                                                           \
    do {                                                                                                     \
        if (lane_count == 8) SANDY_ROPE_LAUNCH(rope_split_lines_kernel, T, U, F, false, 0x141);              \
        else if (lane_count == 16) SANDY_ROPE_LAUNCH(rope_split_lines_kernel, T, U, F, false, 0x140);        \
        else SANDY_ROPE_LAUNCH(rope_split_lines_kernel, T, U, F, false, 0);                                  \
    } while (0)
#define SANDY_ROPE_LINES_F(T, U)                 \
    do {                                         \
        if (full) SANDY_ROPE_LINES(T, U, true);  \
        else SANDY_ROPE_LINES(T, U, false);      \
    } while (0)
#define SANDY_ROPE_LINES_T(T)                          \
    do {                                               \
        if (u == 6) SANDY_ROPE_LINES_F(T, 6);          \
        else if (u == 4) SANDY_ROPE_LINES_F(T, 4);     \
        else if (u == 2) SANDY_ROPE_LINES_F(T, 2);     \
        else SANDY_ROPE_LINES_F(T, 1);                 \
    } while (0)
            if (bf) SANDY_ROPE_LINES_T(BF16);
            else SANDY_ROPE_LINES_T(F32);
#undef SANDY_ROPE_LINES_T
#undef SANDY_ROPE_LINES_F
#undef SANDY_ROPE_LINES
        } else if (split_half) {
            if (bf) SANDY_ROPE_U(rope_split_kernel, BF16);
            else SANDY_ROPE_U(rope_split_kernel, F32);
        } else {
            if (bf) SANDY_ROPE_U(rope_interleaved_kernel, BF16);
            else SANDY_ROPE_U(rope_interleaved_kernel, F32);
        }
#undef SANDY_ROPE_U
#undef SANDY_ROPE_F
#undef SANDY_ROPE_LAUNCH
    } else {
        for (int i = 0; i < n; i++) {
            if (sh[i].total == 0) continue;
            const SandyTensor* x = xs[i];
            const SandyTensor* out = outs[i];
            Strided st{};
            st.rank = x->rank;
            for (int d = 0; d < x->rank; d++) {
                st.dims[d] = x->dims[d];
                st.xs[d] = x->strides[d];
                st.os[d] = out->strides[d];
            }
            const int64_t t = sh[i].vectors * (dim / 2);
            dim3 grid(static_cast<unsigned>((t + 255) / 256));
            hipLaunchKernelGGL(rope_generic_kernel, grid, dim3(256), 0, stream, base_ptr(*x), x->dtype, base_ptr(*out),
                               ids, ids_dt, mode[i], seq, sh[i].vectors, static_cast<int>(dim), rot_pairs,
                               split_half ? 1 : 0, st, args, errw);
        }
    }
    SANDY_HIP_TRY(hipGetLastError(), e, "rope launch");
    return ok(e);
}

} // namespace
} // namespace sandy_hip

extern "C" int sandy_hip_rope(const SandyTensor* x, const SandyTensor* position_ids, double theta,
                              int64_t rotary_dim, int32_t split_half, const SandyTensor* out,
                              void* stream_, char* err, size_t err_cap) {
    const SandyTensor* xs[1] = {x};
    const SandyTensor* outs[1] = {out};
    return rope_run(xs, outs, 1, position_ids, theta, rotary_dim, split_half, static_cast<hipStream_t>(stream_),
                    Err{err, err_cap});
}

extern "C" int sandy_hip_rope_pair(const SandyTensor* q, const SandyTensor* k, const SandyTensor* position_ids,
                                   double theta, int64_t rotary_dim, int32_t split_half, const SandyTensor* q_out,
                                   const SandyTensor* k_out, void* stream_, char* err, size_t err_cap) {
    Err e{err, err_cap};
    if (!valid_rank(q) || !valid_rank(k)) return fail(e, SANDY_ERR_INVALID, "rope tensor rank out of range");
    if (q->dtype != k->dtype) return fail(e, SANDY_ERR_INVALID, "rope pair inputs must have one dtype");
    if (q->rank < 2 || k->rank < 2 || q->dims[q->rank - 1] != k->dims[k->rank - 1] ||
        q->dims[q->rank - 2] != k->dims[k->rank - 2])
        return fail(e, SANDY_ERR_INVALID, "rope pair inputs must share sequence length and last dimension");
    const SandyTensor* xs[2] = {q, k};
    const SandyTensor* outs[2] = {q_out, k_out};
    return rope_run(xs, outs, 2, position_ids, theta, rotary_dim, split_half, static_cast<hipStream_t>(stream_), e);
}

// The cos/sin cache of a forward pass's positions: cache [seq, rotary_dim / 2,
// 2] f32 holds (cos, sin) of position(s) / theta^(2i / d) -- d = dim for
// split-half, rotary_dim for interleaved -- for sequence index s, with the
// positions of sandy_hip_rope (position_ids NULL: s; numel 1: ids[0] + s;
// numel seq: ids[s]).
extern "C" int sandy_hip_rope_cache(const SandyTensor* position_ids, int64_t seq, double theta, int64_t rotary_dim,
                                    int64_t dim, int32_t split_half, const SandyTensor* cache, void* stream_, char* err,
                                    size_t err_cap) {
    Err e{err, err_cap};
    if (!valid_rank(cache)) return fail(e, SANDY_ERR_INVALID, "rope cache tensor rank out of range");
    const float th = static_cast<float>(theta);
    if (th <= 0.0f) return fail(e, SANDY_ERR_INVALID, "rope theta must be > 0");
    if (dim <= 0 || dim % 2 != 0) return fail(e, SANDY_ERR_INVALID, "rope last dimension must be positive and even");
    if (rotary_dim < 0) rotary_dim = dim;
    if (rotary_dim <= 0 || rotary_dim % 2 != 0) return fail(e, SANDY_ERR_INVALID, "rope rotary_dim must be positive and even");
    if (rotary_dim > dim) return fail(e, SANDY_ERR_INVALID, "rope rotary_dim must be <= last dimension");
    if (rotary_dim / 2 > kMaxPairs) return fail(e, SANDY_ERR_UNSUPPORTED, "rope rotary_dim above %d", 2 * kMaxPairs);
    const int rot_pairs = static_cast<int>(rotary_dim / 2);
    if (cache->dtype != SANDY_F32 || cache->rank != 3 || cache->dims[0] != seq || cache->dims[1] != rot_pairs ||
        cache->dims[2] != 2 || !contiguous(*cache))
        return fail(e, SANDY_ERR_INVALID, "rope cache must be a contiguous [seq, rotary_dim / 2, 2] f32 tensor");
    if ((reinterpret_cast<uintptr_t>(base_ptr(*cache)) & 7u) != 0) return fail(e, SANDY_ERR_UNSUPPORTED, "rope cache must be 8-byte aligned");
    int mode = 0;
    if (position_ids) {
        if (!is_index(position_ids->dtype)) return fail(e, SANDY_ERR_INVALID, "rope position_ids must be i32 or i64");
        const int64_t cnt = numel(*position_ids);
        if (cnt != 1 && cnt != seq) return fail(e, SANDY_ERR_INVALID, "rope cache position_ids numel must be 1 or the sequence length");
        if (!contiguous(*position_ids)) return fail(e, SANDY_ERR_UNSUPPORTED, "rope position_ids must be contiguous");
        mode = cnt == 1 && seq != 1 ? 1 : 2;
    }
    if (seq == 0) return ok(e);
    RopeArgs args{};
    const float div = static_cast<float>(split_half ? dim : rotary_dim);
    for (int p = 0; p < rot_pairs; p++) args.denom[p] = std::pow(th, static_cast<float>(2 * p) / div);
    int status = 0;
    uint32_t* errw = device_error_word(e, &status);
    if (status) return status;
    const int64_t n = seq * rot_pairs;
    hipLaunchKernelGGL(rope_cache_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0,
                       static_cast<hipStream_t>(stream_), position_ids ? base_ptr(*position_ids) : nullptr,
                       position_ids ? position_ids->dtype : SANDY_I64, mode, seq, rot_pairs, args, errw,
                       static_cast<float2*>(base_ptr(*cache)));
    SANDY_HIP_TRY(hipGetLastError(), e, "rope cache launch");
    return ok(e);
}

// Split-half RoPE of q (and k, or NULL) from a cos/sin cache built by
// sandy_hip_rope_cache for the same sequence length and head dim: the same
// outputs as sandy_hip_rope_pair with the cache's positions and theta.
extern "C" int sandy_hip_rope_pair_cached(const SandyTensor* q, const SandyTensor* k, const SandyTensor* cache,
                                          const SandyTensor* q_out, const SandyTensor* k_out, void* stream_,
                                          char* err, size_t err_cap) {
    Err e{err, err_cap};
    const int n = k ? 2 : 1;
    const SandyTensor* xs[2] = {q, k};
    const SandyTensor* outs[2] = {q_out, k_out};
    RopeShape sh[2];
    for (int i = 0; i < n; i++) {
        const int st = rope_check(xs[i], outs[i], sh[i], e);
        if (st) return st;
    }
    if (n == 2 && (q->dtype != k->dtype || sh[0].seq != sh[1].seq || sh[0].dim != sh[1].dim))
        return fail(e, SANDY_ERR_INVALID, "rope pair inputs must share sequence length and last dimension");
    if (!valid_rank(cache) || cache->dtype != SANDY_F32 || cache->rank != 3 || cache->dims[0] != sh[0].seq ||
        cache->dims[2] != 2 || !contiguous(*cache) || cache->dims[1] <= 0 || 2 * cache->dims[1] > sh[0].dim)
        return fail(e, SANDY_ERR_INVALID, "rope cache must be a contiguous [seq, rotary_dim / 2, 2] f32 tensor");
    const int64_t seq = sh[0].seq, dim = sh[0].dim;
    const int rot_pairs = static_cast<int>(cache->dims[1]);
    const int chunks = static_cast<int>(dim / 16);
    bool ok_shape = dim % 16 == 0 && chunks <= 32 && (chunks & (chunks - 1)) == 0 &&
                    (reinterpret_cast<uintptr_t>(base_ptr(*cache)) & 7u) == 0;
    int64_t outer = 0;
    for (int i = 0; i < n; i++) {
        const uintptr_t a = reinterpret_cast<uintptr_t>(base_ptr(*xs[i])) | reinterpret_cast<uintptr_t>(base_ptr(*outs[i]));
        ok_shape = ok_shape && contiguous(*xs[i]) && contiguous(*outs[i]) && (a & 15u) == 0;
        outer += sh[i].outer;
    }
    if (!ok_shape)
        return fail(e, SANDY_ERR_UNSUPPORTED,
                    "rope from a cache takes contiguous 16-byte aligned split-half rows whose half is a power-of-two "
                    "multiple of 8 elements (up to 256)");
    if (outer == 0 || seq == 0) return ok(e);
    int status = 0;
    uint32_t* errw = device_error_word(e, &status);
    if (status) return status;
    // head groups as the direct kernel: 6 heads when they divide by 6, else
    // the largest of 4 / 2 / 1 that divides the heads
    const int per = outer % 6 == 0 ? 6 : outer % 4 == 0 ? 4 : outer % 2 == 0 ? 2 : 1;
    const int groups = static_cast<int>(outer / per);
    const int64_t threads = seq * 2 * chunks * groups;
    if (threads + 255 >= (int64_t(1) << 31)) return fail(e, SANDY_ERR_UNSUPPORTED, "rope from a cache: tensor too large");
    const bool full = rot_pairs == dim / 2;
    RopeArgs args{};
    const void* px = base_ptr(*q);
    void* po = base_ptr(*q_out);
    const void* px2 = n == 2 ? base_ptr(*k) : px;
    void* po2 = n == 2 ? base_ptr(*k_out) : po;
    const float2* tab = static_cast<const float2*>(base_ptr(*cache));
    dim3 grid(static_cast<unsigned>((threads + 255) / 256));
    hipStream_t stream = static_cast<hipStream_t>(stream_);
#define SANDY_ROPE_TAB_X(T, U, F, X)                                                                                \
    hipLaunchKernelGGL((rope_split_lines_kernel<T, U, F, true, X>), grid, dim3(256), 0, stream, px, po, px2, po2,  \
                       sh[0].outer, nullptr, SANDY_I64, 0, seq, outer, static_cast<int>(dim), rot_pairs, groups, per, \
                       args, errw, tab)
#define SANDY_ROPE_TAB(T, U, F)                                    \
    do {                                                           \
        if (chunks == 4) SANDY_ROPE_TAB_X(T, U, F, 0x141);         \
        else if (chunks == 8) SANDY_ROPE_TAB_X(T, U, F, 0x140);    \
        else SANDY_ROPE_TAB_X(T, U, F, 0);                         \
    } while (0)
#define SANDY_ROPE_TAB_F(T, U)                 \
    do {                                       \
        if (full) SANDY_ROPE_TAB(T, U, true);  \
        else SANDY_ROPE_TAB(T, U, false);      \
    } while (0)
#define SANDY_ROPE_TAB_T(T)                      \
    do {                                         \
        if (per == 6) SANDY_ROPE_TAB_F(T, 6);    \
        else if (per == 4) SANDY_ROPE_TAB_F(T, 4); \
        else if (per == 2) SANDY_ROPE_TAB_F(T, 2); \
        else SANDY_ROPE_TAB_F(T, 1);             \
    } while (0)
    if (q->dtype == SANDY_BF16) SANDY_ROPE_TAB_T(BF16);
    else SANDY_ROPE_TAB_T(F32);
#undef SANDY_ROPE_TAB_T
#undef SANDY_ROPE_TAB_F
#undef SANDY_ROPE_TAB
#undef SANDY_ROPE_TAB_X
    SANDY_HIP_TRY(hipGetLastError(), e, "rope launch");
    return ok(e);
}
