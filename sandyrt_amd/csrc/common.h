// common.h -- shared host/device helpers of the gfx950 backend.
//
// Host side: error reporting into the caller's buffer, SandyTensor checks,
// the per-device sticky error word and the per-device workspace.
// Device side: bf16 <-> f32 with the reference's rounding, 128-bit vector
// loads/stores of 8 elements, wave64 reductions.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <cstdlib>
#include <cstdio>
#include <cstring>
#include <string>

#include "../../include/sandyrt_hip.h"

namespace sandy_hip {

// ---------------------------------------------------------------- host errors
struct Err {
    char* buf;
    size_t cap;
};

inline int fail(Err e, int code, const char* fmt, ...) {
    if (e.buf && e.cap) {
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(e.buf, e.cap, fmt, ap);
        va_end(ap);
    }
    return code;
}

inline int ok(Err e) {
    if (e.buf && e.cap) e.buf[0] = 0;
    return SANDY_OK;
}

#define SANDY_HIP_TRY(expr, e, what)                                                   \
    do {                                                                               \
        hipError_t st_ = (expr);                                                       \
        if (st_ != hipSuccess)                                                         \
            return ::sandy_hip::fail(e, SANDY_ERR_HIP, "%s: %s", what, hipGetErrorString(st_)); \
    } while (0)

// ---------------------------------------------------------------- tensor helpers
inline int64_t numel(const SandyTensor& t) {
    int64_t n = 1;
    for (int i = 0; i < t.rank; i++) n *= t.dims[i];
    return n;
}

inline bool contiguous(const SandyTensor& t) {
    for (int i = 0; i < t.rank; i++)
        if (t.dims[i] == 0) return true;  // empty: no element is addressed
    int64_t s = 1;
    for (int i = t.rank - 1; i >= 0; i--) {
        if (t.dims[i] != 1 && t.strides[i] != s) return false;
        s *= t.dims[i];
    }
    return true;
}

inline bool same_shape(const SandyTensor& a, const SandyTensor& b) {
    if (a.rank != b.rank) return false;
    for (int i = 0; i < a.rank; i++)
        if (a.dims[i] != b.dims[i]) return false;
    return true;
}

// Integer value of an environment switch (measurement and test selection of
// kernel forms), or dflt when unset or empty.
inline int env_int(const char* name, int dflt) {
    const char* v = std::getenv(name);
    return v && *v ? std::atoi(v) : dflt;
}

inline bool is_float(int32_t dt) { return dt == SANDY_F32 || dt == SANDY_BF16; }
inline bool is_index(int32_t dt) { return dt == SANDY_I32 || dt == SANDY_I64; }
inline size_t dtype_size(int32_t dt) {
    switch (dt) {
        case SANDY_F32: return 4;
        case SANDY_F16: return 2;
        case SANDY_BF16: return 2;
        case SANDY_I32: return 4;
        case SANDY_I64: return 8;
        case SANDY_U8: return 1;
    }
    return 0;
}

// Element address of storage_offset (data + offset * element size).
inline void* base_ptr(const SandyTensor& t) {
    return static_cast<char*>(t.data) + t.storage_offset * static_cast<int64_t>(dtype_size(t.dtype));
}

inline bool valid_rank(const SandyTensor* t) { return t && t->rank >= 0 && t->rank <= SANDY_HIP_MAX_RANK; }

// Per-device sticky error word (one uint32 in device memory, zeroed at
// creation).  Kernels atomicOr SandyDeviceError bits into it.
uint32_t* device_error_word(Err e, int* status);

// Workspace slots kPagedStageSlot0 .. + SANDY_HIP_PAGED_STAGE_SLOTS - 1 hold
// staged paged operands (paged_operand.hip); slots below it belong to the
// kernels' own scratch.
constexpr int kPagedStageSlot0 = 8;

// Per-device, per-purpose grow-only scratch.  The returned memory stays valid
// until the next call with the same slot and a larger size; callers that
// need zeroed memory keep it zero themselves.
void* device_workspace(int slot, size_t bytes, hipStream_t stream, Err e, int* status);

// Zero-initialised per-device counters; zeroed when (re)allocated, kept zero
// afterwards by the kernels that use them.
void* device_counters(int slot, size_t bytes, hipStream_t stream, Err e, int* status);


// ---------------------------------------------------------------- device helpers
__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __uint_as_float(static_cast<uint32_t>(b) << 16); }

// round to nearest even, NaN not special-cased (src/core/Tensor.h:43-49)
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
    uint32_t u = __float_as_uint(f);
    return static_cast<uint16_t>((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    return static_cast<uint32_t>(f32_to_bf16(lo)) | (static_cast<uint32_t>(f32_to_bf16(hi)) << 16);
}

struct BF16 {};
struct F32 {};

// Eight consecutive elements <-> eight floats (16 B for bf16, 32 B for f32).
template <typename T>
struct Vec8;

template <>
struct Vec8<BF16> {
    using elem = uint16_t;
    // raw 16-byte chunk: load early, unpack only when the values are needed,
    // so independent work can run while the load is in flight
    using raw = uint4;
    __device__ __forceinline__ static raw load_raw(const void* p, int64_t i) {
        return *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(p) + i);
    }
    // streamed input read once: non-temporal, so it does not displace reused data
    __device__ __forceinline__ static raw load_raw_nt(const void* p, int64_t i) {
        typedef unsigned int u32x4_nt __attribute__((ext_vector_type(4)));
        const u32x4_nt v = __builtin_nontemporal_load(
                reinterpret_cast<const u32x4_nt*>(static_cast<const uint16_t*>(p) + i));
        return uint4{v.x, v.y, v.z, v.w};
    }
    __device__ __forceinline__ static void unpack(const raw& r, float (&v)[8]) {
        const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
        for (int j = 0; j < 4; j++) {
            v[2 * j] = __uint_as_float(w[j] << 16);
            v[2 * j + 1] = __uint_as_float(w[j] & 0xffff0000u);
        }
    }
    __device__ __forceinline__ static void load(const void* p, int64_t i, float (&v)[8]) {
        uint4 r = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(p) + i);
        uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
        for (int j = 0; j < 4; j++) {
            v[2 * j] = __uint_as_float(w[j] << 16);
            v[2 * j + 1] = __uint_as_float(w[j] & 0xffff0000u);
        }
    }
    __device__ __forceinline__ static void store(void* p, int64_t i, const float (&v)[8]) {
        uint4 r;
        r.x = pack_bf16x2(v[0], v[1]);
        r.y = pack_bf16x2(v[2], v[3]);
        r.z = pack_bf16x2(v[4], v[5]);
        r.w = pack_bf16x2(v[6], v[7]);
        // streamed output: non-temporal, so it does not sit dirty in L2 until the
        // end-of-kernel write-back (measured: shorter kernel tails on gfx950)
        typedef unsigned int u32x4_nt __attribute__((ext_vector_type(4)));
        __builtin_nontemporal_store(u32x4_nt{r.x, r.y, r.z, r.w},
                                    reinterpret_cast<u32x4_nt*>(static_cast<uint16_t*>(p) + i));
    }
    // value as it will read back after a store (rounded to bf16)
    __device__ __forceinline__ static float round(float f) { return bf16_to_f32(f32_to_bf16(f)); }
    __device__ __forceinline__ static float load1(const void* p, int64_t i) {
        return bf16_to_f32(static_cast<const uint16_t*>(p)[i]);
    }
    __device__ __forceinline__ static void store1(void* p, int64_t i, float f) {
        static_cast<uint16_t*>(p)[i] = f32_to_bf16(f);
    }
};

template <>
struct Vec8<F32> {
    using elem = float;
    struct raw {
        float4 a, b;
    };
    __device__ __forceinline__ static raw load_raw(const void* p, int64_t i) {
        const float4* q = reinterpret_cast<const float4*>(static_cast<const float*>(p) + i);
        return raw{q[0], q[1]};
    }
    __device__ __forceinline__ static raw load_raw_nt(const void* p, int64_t i) {
        typedef float f32x4_nt __attribute__((ext_vector_type(4)));
        const f32x4_nt* q = reinterpret_cast<const f32x4_nt*>(static_cast<const float*>(p) + i);
        const f32x4_nt a = __builtin_nontemporal_load(q), b = __builtin_nontemporal_load(q + 1);
        return raw{float4{a.x, a.y, a.z, a.w}, float4{b.x, b.y, b.z, b.w}};
    }
    __device__ __forceinline__ static void unpack(const raw& r, float (&v)[8]) {
        v[0] = r.a.x; v[1] = r.a.y; v[2] = r.a.z; v[3] = r.a.w;
        v[4] = r.b.x; v[5] = r.b.y; v[6] = r.b.z; v[7] = r.b.w;
    }
    __device__ __forceinline__ static void load(const void* p, int64_t i, float (&v)[8]) {
        const float4* q = reinterpret_cast<const float4*>(static_cast<const float*>(p) + i);
        float4 a = q[0], b = q[1];
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
        v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    }
    __device__ __forceinline__ static void store(void* p, int64_t i, const float (&v)[8]) {
        typedef float f32x4_nt __attribute__((ext_vector_type(4)));  // streamed output, as for bf16
        f32x4_nt* q = reinterpret_cast<f32x4_nt*>(static_cast<float*>(p) + i);
        __builtin_nontemporal_store(f32x4_nt{v[0], v[1], v[2], v[3]}, q);
        __builtin_nontemporal_store(f32x4_nt{v[4], v[5], v[6], v[7]}, q + 1);
    }
    __device__ __forceinline__ static float round(float f) { return f; }
    __device__ __forceinline__ static float load1(const void* p, int64_t i) { return static_cast<const float*>(p)[i]; }
    __device__ __forceinline__ static void store1(void* p, int64_t i, float f) { static_cast<float*>(p)[i] = f; }
};

__device__ __forceinline__ float load_any(const void* p, int32_t dt, int64_t i) {
    return dt == SANDY_BF16 ? Vec8<BF16>::load1(p, i) : Vec8<F32>::load1(p, i);
}
__device__ __forceinline__ void store_any(void* p, int32_t dt, int64_t i, float f) {
    if (dt == SANDY_BF16)
        Vec8<BF16>::store1(p, i, f);
    else
        Vec8<F32>::store1(p, i, f);
}
__device__ __forceinline__ int64_t load_index(const void* p, int32_t dt, int64_t i) {
    return dt == SANDY_I32 ? static_cast<int64_t>(static_cast<const int32_t*>(p)[i]) : static_cast<const int64_t*>(p)[i];
}
__device__ __forceinline__ void store_index(void* p, int32_t dt, int64_t i, int64_t v) {
    if (dt == SANDY_I32)
        static_cast<int32_t*>(p)[i] = static_cast<int32_t>(v);
    else
        static_cast<int64_t*>(p)[i] = v;
}

// sin and cos of a float angle (RoPE): double-precision Cody-Waite reduction
// to [-pi/4, pi/4] with pi/2 split in two doubles (exact for |a| < 2^20),
// Taylor polynomials to r^11 / r^12 in float, quadrant select.  Within 1 ulp
// of the correctly rounded values, like the CPU's sinf/cosf.
__device__ __forceinline__ void rope_sincos(float a, float* s, float* c) {
    const double k = __builtin_rint(static_cast<double>(a) * 0.63661977236758134308);  // 2 / pi
    double rd = fma(-k, 1.5707963267948966192, static_cast<double>(a));               // pi/2 (head)
    rd = fma(-k, 6.123233995736766036e-17, rd);                                        // pi/2 (tail)
    const float r = static_cast<float>(rd);
    const float r2 = r * r;
    float sp = fmaf(r2, -2.5052108385441718775e-8f, 2.7557319223985890653e-6f);   // -1/11!, 1/9!
    sp = fmaf(r2, sp, -1.9841269841269841270e-4f);                                 // -1/7!
    sp = fmaf(r2, sp, 8.3333333333333333333e-3f);                                  // 1/5!
    sp = fmaf(r2, sp, -1.6666666666666666667e-1f);                                 // -1/3!
    const float sv = fmaf(r * r2, sp, r);
    float cp = fmaf(r2, 2.0876756987868098979e-9f, -2.7557319223985890653e-7f);   // 1/12!, -1/10!
    cp = fmaf(r2, cp, 2.4801587301587301587e-5f);                                  // 1/8!
    cp = fmaf(r2, cp, -1.3888888888888888889e-3f);                                 // -1/6!
    cp = fmaf(r2, cp, 4.1666666666666666667e-2f);                                  // 1/4!
    cp = fmaf(r2, cp, -0.5f);
    const float cv = fmaf(r2, cp, 1.0f);
    const int q = static_cast<int>(k);
    float ss = (q & 1) ? cv : sv;
    float cc = (q & 1) ? sv : cv;
    if (q & 2) ss = -ss;
    if ((q + 1) & 2) cc = -cc;
    *s = ss;
    *c = cc;
}

// tanh in a few VALU instructions: the odd Taylor series of tanh to y^11
// for |y| < 0.4 (the next term, 21844 y^13 / 6081075, is below 3e-8 of the
// result there), else tanh|y| = 1 - 2 / (e^(2|y|) + 1) with the hardware
// exp2 and reciprocal (relative error below 3e-7 for |y| >= 0.4; 1 past
// |y| = 9.1).  The same code is compiled into the generated element-wise
// groups, so fused and unfused gated activations agree bit for bit.
__device__ __forceinline__ float sandy_tanh(float y) {
    const float a = fabsf(y);
    if (a < 0.4f) {
        const float y2 = y * y;
        float p = fmaf(y2, -0.008863235529902197f, 0.021869488536155203f);
        p = fmaf(y2, p, -0.05396825396825397f);
        p = fmaf(y2, p, 0.13333333333333333f);
        p = fmaf(y2, p, -0.3333333333333333f);
        return fmaf(y * y2, p, y);
    }
    const float e = __builtin_amdgcn_exp2f(2.8853900817779268f * a);
    return copysignf(fmaf(-2.0f, __builtin_amdgcn_rcpf(e + 1.0f), 1.0f), y);
}

// h * (1 + tanh(h)) -- the tail of the SiLU node chain (x * sigmoid(x) with
// h = x / 2) -- by the identity 1 + tanh(h) = 2 / (1 + e^(-2h)): 2h / (1 +
// e^(-2h)) with the hardware exp2 and reciprocal, about 3e-7 relative
// everywhere (no cancellation: the denominator is at least 1) in four VALU
// operations instead of tanh's two branches; -inf side -> -0, +inf side ->
// 2h.  The element-wise generator emits it for that node pattern and the
// gated GEMM epilogue calls it, so fused and unfused SiLU agree bit for bit.
__device__ __forceinline__ float sandy_silu_half(float h) {
    return (h + h) * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-2.8853900817779268f * h));
}

// Sum over aligned groups of G lanes (G = 2, 4, 8 or 16) with DPP lane moves
// (quad swaps, then the half-row and row mirrors): every lane of a group ends
// with the group's total.  ALU-latency moves, unlike __shfl_xor's LDS
// crossbar; doubles move as two 32-bit halves.
template <int CTRL>
__device__ __forceinline__ double dpp_move(double v) {
    const uint64_t u = static_cast<uint64_t>(__double_as_longlong(v));
    const int lo = __builtin_amdgcn_update_dpp(0, static_cast<int>(static_cast<uint32_t>(u)), CTRL, 0xf, 0xf, false);
    const int hi = __builtin_amdgcn_update_dpp(0, static_cast<int>(static_cast<uint32_t>(u >> 32)), CTRL, 0xf, 0xf, false);
    return __longlong_as_double(static_cast<long long>((static_cast<uint64_t>(static_cast<uint32_t>(hi)) << 32) |
                                                       static_cast<uint32_t>(lo)));
}

// the value of lane ^ 1 (quad_perm [1, 0, 3, 2]), a VALU move
__device__ __forceinline__ float lane_xor1(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xf, 0xf, false));
}

template <int G>
__device__ __forceinline__ double group_sum(double v) {
    static_assert(G == 2 || G == 4 || G == 8 || G == 16, "group of 2, 4, 8 or 16 lanes");
    v += dpp_move<0xB1>(v);                     // quad_perm [1, 0, 3, 2]: lane ^ 1
    if constexpr (G >= 4) v += dpp_move<0x4E>(v);   // quad_perm [2, 3, 0, 1]: lane ^ 2
    if constexpr (G >= 8) v += dpp_move<0x141>(v);  // row_half_mirror: quad 0 <-> quad 1
    if constexpr (G >= 16) v += dpp_move<0x140>(v); // row_mirror: half row 0 <-> 1
    return v;
}

// wave64 butterfly reductions (every lane ends with the full result)
template <typename T>
__device__ __forceinline__ T wave_sum(T v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
    return v;
}

// Lane l combined with lane l ^ 16 (or l ^ 32) through gfx950's
// v_permlane16_swap / v_permlane32_swap: with both operands v, the pair
// returned holds v[l & ~16] and v[l | 16] (v[l & 31] and v[l | 32]), so one
// VALU exchange replaces an LDS-routed ds_bpermute.  The result is the same
// in both lanes of a pair (max and + are commutative).
__device__ __forceinline__ float max_xor16(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float max_xor32(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_xor16(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float sum_xor32(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

constexpr int kWave = 64;

} // namespace sandy_hip
