// elementwise.hip -- fused element-wise groups (ElementwiseKernelOp) as
// generated gfx950 code.
//
// The reference interprets the scalar DAG per element in one generic CUDA
// kernel (src/device/cuda/CudaElementwiseKernels.cu:117-213): a switch per
// node, one element per thread, int64 div/mod per strided or broadcast load,
// no vector loads.  Here each distinct DAG (ops, constants, input dtypes and
// access modes) becomes straight-line HIP C++ that hipRTC compiles for gfx950
// on first use; the code object is cached per device by the source text.
//
// Node semantics are the reference's: every scalar is an fp32 value, Load
// converts the input element to fp32, Constant is (float)constant, Cast passes
// through, and the result is stored once in the output dtype (bf16 with the
// reference's round-to-nearest-even).  Rsqrt is emitted as 1 / sqrtf(a)
// (correctly rounded) rather than a hardware approximation.  Arithmetic is
// compiled without FMA contraction so a * b + c keeps the reference's two
// roundings.
//
// Access modes per input: same-shape contiguous, right-aligned broadcast
// (element index = linear % numel, CudaElementwiseKernels.cu:171-174), scalar
// (numel 1) or strided (dims/strides passed at launch).  When the output and
// every input allow it, threads walk the tensor in 8-element chunks with
// 128-bit loads and stores, two chunks in flight per thread (one below 2^20
// elements) over a grid of at most 4096 workgroups; contiguous inputs are
// read non-temporally (streamed once; broadcast inputs are re-read and stay
// cached).  Otherwise one element per thread.
#include "common.h"

#include <hip/hiprtc.h>

#include <algorithm>
#include <map>
#include <mutex>
#include <sstream>
#include <string>
#include <vector>

namespace sandy_hip {
namespace {

enum Mode { kContig = 0, kBroadcast = 1, kScalar = 2, kStrided = 3 };

struct EwArgs {
    const void* in[SANDY_HIP_MAX_INPUTS];
    int64_t numel[SANDY_HIP_MAX_INPUTS];
    int64_t dims[SANDY_HIP_MAX_INPUTS][SANDY_HIP_MAX_RANK];
    int64_t strides[SANDY_HIP_MAX_INPUTS][SANDY_HIP_MAX_RANK];
    int32_t rank[SANDY_HIP_MAX_INPUTS];
    void* out;
    int64_t n;
    int64_t odims[SANDY_HIP_MAX_RANK];
    int64_t ostrides[SANDY_HIP_MAX_RANK];
    int32_t orank;
};

// The vectorised kernel reads only pointers and element counts: a 144-byte
// argument block instead of the 1.2 KB one the strided kernel needs.
struct EwVecArgs {
    const void* in[SANDY_HIP_MAX_INPUTS];
    int64_t numel[SANDY_HIP_MAX_INPUTS];
    void* out;
    int64_t n;
};

// The generated code declares the same struct layout.
const char* kPrelude = R"(
typedef unsigned short u16;
typedef long long i64;
struct EwArgs {
  const void* in[8]; i64 numel[8]; i64 dims[8][8]; i64 strides[8][8]; int rank[8];
  void* out; i64 n; i64 odims[8]; i64 ostrides[8]; int orank;
};
struct EwVecArgs { const void* in[8]; i64 numel[8]; void* out; i64 n; };
__device__ __forceinline__ float bf2f(u16 b) { return __uint_as_float(((unsigned)b) << 16); }
__device__ __forceinline__ u16 f2bf(float f) { unsigned u = __float_as_uint(f); return (u16)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16); }
// two values in one v_cvt_pk_bf16_f32: round to nearest even like f2bf for every
// value but a NaN (kept a NaN, where f2bf can carry some NaN payloads into -0 or inf)
typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));
typedef float f32x2v __attribute__((ext_vector_type(2)));
__device__ __forceinline__ unsigned pk2bf(float lo, float hi) {
  return __builtin_bit_cast(unsigned, __builtin_convertvector(f32x2v{lo, hi}, bf16x2v));
}
__device__ __forceinline__ i64 strided_index(const i64* dims, const i64* strides, int rank, i64 lin) {
  i64 off = 0;
  for (int d = rank - 1; d >= 0; d--) { i64 c = lin % dims[d]; lin /= dims[d]; off += c * strides[d]; }
  return off;
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
// h * (1 + tanh(h)) as 2h / (1 + e^(-2h)): the same code as the library's
// sandy_silu_half (common.h), emitted for the SiLU node pattern
__device__ __forceinline__ float sandy_silu_half(float h) {
  return (h + h) * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-2.8853900817779268f * h));
}
__device__ __forceinline__ void ld8_bf16(const void* p, i64 i, float* v) {
  uint4 r = *(const uint4*)((const u16*)p + i);
  unsigned w[4] = {r.x, r.y, r.z, r.w};
  for (int j = 0; j < 4; j++) { v[2*j] = __uint_as_float(w[j] << 16); v[2*j+1] = __uint_as_float(w[j] & 0xffff0000u); }
}
__device__ __forceinline__ void ldnt8_bf16(const void* p, i64 i, float* v) {
  typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
  u32x4 r = __builtin_nontemporal_load((const u32x4*)((const u16*)p + i));
  unsigned w[4] = {r.x, r.y, r.z, r.w};
  for (int j = 0; j < 4; j++) { v[2*j] = __uint_as_float(w[j] << 16); v[2*j+1] = __uint_as_float(w[j] & 0xffff0000u); }
}
__device__ __forceinline__ void ldnt8_f32(const void* p, i64 i, float* v) {
  typedef float f32x4 __attribute__((ext_vector_type(4)));
  const f32x4* q = (const f32x4*)((const float*)p + i);
  f32x4 a = __builtin_nontemporal_load(q), b = __builtin_nontemporal_load(q + 1);
  v[0]=a.x; v[1]=a.y; v[2]=a.z; v[3]=a.w; v[4]=b.x; v[5]=b.y; v[6]=b.z; v[7]=b.w;
}
__device__ __forceinline__ void ld8_f32(const void* p, i64 i, float* v) {
  const float4* q = (const float4*)((const float*)p + i); float4 a = q[0], b = q[1];
  v[0]=a.x; v[1]=a.y; v[2]=a.z; v[3]=a.w; v[4]=b.x; v[5]=b.y; v[6]=b.z; v[7]=b.w;
}
__device__ __forceinline__ void st8_bf16(void* p, i64 i, const float* v) {
  uint4 r;
  r.x = pk2bf(v[0], v[1]);
  r.y = pk2bf(v[2], v[3]);
  r.z = pk2bf(v[4], v[5]);
  r.w = pk2bf(v[6], v[7]);
  typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
  __builtin_nontemporal_store(u32x4{r.x, r.y, r.z, r.w}, (u32x4*)((u16*)p + i));
}
__device__ __forceinline__ void st8_f32(void* p, i64 i, const float* v) {
  typedef float f32x4 __attribute__((ext_vector_type(4)));
  f32x4* q = (f32x4*)((float*)p + i);
  __builtin_nontemporal_store(f32x4{v[0], v[1], v[2], v[3]}, q);
  __builtin_nontemporal_store(f32x4{v[4], v[5], v[6], v[7]}, q + 1);
}
)";

std::string float_literal(double c) {
    float f = static_cast<float>(c);
    uint32_t bits;
    std::memcpy(&bits, &f, 4);
    std::ostringstream os;
    os << "__uint_as_float(0x" << std::hex << bits << "u)";
    return os.str();
}

std::string node_expr(const SandyScalarNode& n) {
    auto a = "s" + std::to_string(n.operands[0]);
    auto b = n.operand_count > 1 ? "s" + std::to_string(n.operands[1]) : std::string();
    switch (n.op) {
        case 1: return float_literal(n.constant);
        case 2: return "__fadd_rn(" + a + ", " + b + ")";
        case 3: return "__fsub_rn(" + a + ", " + b + ")";
        case 4: return "__fmul_rn(" + a + ", " + b + ")";
        case 5: return "__fdiv_rn(" + a + ", " + b + ")";
        case 6: return "fmaxf(" + a + ", " + b + ")";
        case 7: return "fminf(" + a + ", " + b + ")";
        case 8: return "(-" + a + ")";
        case 9: return "sqrtf(" + a + ")";
        case 10: return "__fdiv_rn(1.0f, sqrtf(" + a + "))";
        case 11: return "expf(" + a + ")";
        case 12: return "logf(" + a + ")";
        case 13: return "sandy_tanh(" + a + ")";
        case 14: return "fmaxf(" + a + ", 0.0f)";
        case 15: return a;
    }
    return "0.0f";
}

// The SiLU tail h * (1 + tanh(h)) of the reference's lowering (x * sigmoid(x)
// as (x / 2)(1 + tanh(x / 2)), src/ir/BuiltinLowering.cpp:142-158): for a MUL
// node whose operands are h and ADD(CONST 1, TANH(h)) (either order), the
// id of h, else -1.  Such a node is emitted as sandy_silu_half(h).
int64_t silu_tail_of(const SandyScalarNode* nodes, int count, const SandyScalarNode& n) {
    if (n.op != 4 || n.operand_count != 2) return -1;
    auto find = [&](uint32_t id) -> const SandyScalarNode* {
        for (int i = 0; i < count; i++)
            if (nodes[i].id == id) return &nodes[i];
        return nullptr;
    };
    for (int side = 0; side < 2; side++) {
        const uint32_t h = n.operands[side];
        const SandyScalarNode* a = find(n.operands[1 - side]);
        if (!a || a->op != 2 || a->operand_count != 2) continue;
        for (int as = 0; as < 2; as++) {
            const SandyScalarNode* c = find(a->operands[as]);
            const SandyScalarNode* t = find(a->operands[1 - as]);
            if (c && t && c->op == 1 && static_cast<float>(c->constant) == 1.0f && t->op == 13 &&
                t->operand_count == 1 && t->operands[0] == h)
                return h;
        }
    }
    return -1;
}

// chunks of 8 elements per thread per grid stride of the vectorised kernel:
// one below 2^20 elements, where twice the workgroups beat two chunks in
// flight per thread (GeGLU [64, 10240]: 3.55 -> 3.04 us), two above
// (SwiGLU [4096, 704]: 4.8 vs 5.4 us with one; four is slower everywhere)
int vec_chunks(int64_t n) { return n < (int64_t{1} << 20) ? 1 : 2; }

std::string generate(const SandyScalarNode* nodes, int count, uint32_t result, const int32_t* in_dt,
                     const int* modes, int nin, int32_t out_dt, bool vec, int U) {
    std::ostringstream s;
    s << kPrelude;
    s << "extern \"C\" __global__ __launch_bounds__(256) void sandy_ew(" << (vec ? "EwVecArgs" : "EwArgs")
      << " a) {\n";
    if (vec) {
        // chunk j of 8 elements; a thread takes chunks c, c + 256, ... of each
        // (256 U)-chunk stride of the grid, all U chunks' loads issued first
        s << "  const i64 chunks = a.n >> 3;\n";
        s << "  for (i64 c0 = (i64)blockIdx.x * " << 256 * U << " + threadIdx.x; c0 < chunks; c0 += (i64)gridDim.x * "
          << 256 * U << ") {\n";
        for (int u = 0; u < U; u++) {
            const std::string cidx = "(c0 + " + std::to_string(256 * u) + ")";
            for (int i = 0; i < nin; i++) s << "    float in" << i << "_" << u << "[8];\n";
            if (u > 0) s << "    if (" << cidx << " < chunks) {\n";
            for (int i = 0; i < nin; i++) {
                const std::string nm = "in" + std::to_string(i) + "_" + std::to_string(u);
                if (modes[i] == kContig)
                    s << "    " << (in_dt[i] == SANDY_BF16 ? "ldnt8_bf16" : "ldnt8_f32") << "(a.in[" << i << "], "
                      << cidx << " * 8, " << nm << ");\n";
                else if (modes[i] == kBroadcast)
                    s << "    " << (in_dt[i] == SANDY_BF16 ? "ld8_bf16" : "ld8_f32") << "(a.in[" << i << "], ("
                      << cidx << " * 8) % a.numel[" << i << "], " << nm << ");\n";
                else  // scalar
                    s << "    { float v = " << (in_dt[i] == SANDY_BF16 ? "bf2f(((const u16*)a.in[" : "(((const float*)a.in[")
                      << i << "])[0]); for (int k = 0; k < 8; k++) " << nm << "[k] = v; }\n";
            }
            if (u > 0) s << "    }\n";
        }
        for (int u = 0; u < U; u++) {
            const std::string cidx = "(c0 + " + std::to_string(256 * u) + ")";
            const std::string suf = "_" + std::to_string(u);
            if (u > 0) s << "    if (" << cidx << " >= chunks) break;\n";
            s << "    {\n    float r[8];\n#pragma unroll\n    for (int k = 0; k < 8; k++) {\n";
            for (int j = 0; j < count; j++) {
                const auto& n = nodes[j];
                s << "      const float s" << n.id << " = ";
                if (n.op == 0) s << "in" << n.input_index << suf << "[k];\n";
                else if (silu_tail_of(nodes, count, n) >= 0) s << "sandy_silu_half(s" << silu_tail_of(nodes, count, n) << ");\n";
                else s << node_expr(n) << ";\n";
            }
            s << "      r[k] = s" << result << ";\n    }\n";
            s << "    " << (out_dt == SANDY_BF16 ? "st8_bf16" : "st8_f32") << "(a.out, " << cidx
              << " * 8, r);\n    }\n";
        }
        s << "  }\n}\n";
    } else {
        s << "  i64 lin = (i64)blockIdx.x * 256 + threadIdx.x;\n  if (lin >= a.n) return;\n";
        for (int i = 0; i < nin; i++) {
            std::string idx;
            if (modes[i] == kContig) idx = "lin";
            else if (modes[i] == kBroadcast) idx = "(a.numel[" + std::to_string(i) + "] ? lin % a.numel[" + std::to_string(i) + "] : 0)";
            else if (modes[i] == kScalar) idx = "0";
            else idx = "strided_index(a.dims[" + std::to_string(i) + "], a.strides[" + std::to_string(i) + "], a.rank[" +
                       std::to_string(i) + "], lin)";
            s << "  const float in" << i << " = ";
            if (in_dt[i] == SANDY_BF16) s << "bf2f(((const u16*)a.in[" << i << "])[" << idx << "]);\n";
            else s << "((const float*)a.in[" << i << "])[" << idx << "];\n";
        }
        for (int j = 0; j < count; j++) {
            const auto& n = nodes[j];
            s << "  const float s" << n.id << " = ";
            if (n.op == 0) s << "in" << n.input_index << ";\n";
            else if (silu_tail_of(nodes, count, n) >= 0) s << "sandy_silu_half(s" << silu_tail_of(nodes, count, n) << ");\n";
            else s << node_expr(n) << ";\n";
        }
        s << "  const i64 o = strided_index(a.odims, a.ostrides, a.orank, lin);\n";
        if (out_dt == SANDY_BF16) s << "  ((u16*)a.out)[o] = f2bf(s" << result << ");\n}\n";
        else s << "  ((float*)a.out)[o] = s" << result << ";\n}\n";
    }
    return s.str();
}

struct Compiled {
    hipModule_t module = nullptr;
    hipFunction_t fn = nullptr;
};

std::mutex g_mu;
std::map<std::pair<int, std::string>, Compiled> g_cache;

int compile(const std::string& src, Compiled* out, Err e) {
    hiprtcProgram prog;
    if (hiprtcCreateProgram(&prog, src.c_str(), "sandy_ew.hip", 0, nullptr, nullptr) != HIPRTC_SUCCESS)
        return fail(e, SANDY_ERR_COMPILE, "hiprtcCreateProgram failed");
    const char* opts[] = {"--offload-arch=gfx950", "-O3", "-ffp-contract=off", "-std=c++17",
                          "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"};
    hiprtcResult rc = hiprtcCompileProgram(prog, sizeof(opts) / sizeof(opts[0]), opts);
    if (rc != HIPRTC_SUCCESS) {
        size_t log_size = 0;
        hiprtcGetProgramLogSize(prog, &log_size);
        std::string log(log_size, '\0');
        if (log_size) hiprtcGetProgramLog(prog, &log[0]);
        hiprtcDestroyProgram(&prog);
        return fail(e, SANDY_ERR_COMPILE, "hipRTC compile of fused group failed: %s", log.substr(0, 400).c_str());
    }
    size_t code_size = 0;
    hiprtcGetCodeSize(prog, &code_size);
    std::vector<char> code(code_size);
    hiprtcGetCode(prog, code.data());
    hiprtcDestroyProgram(&prog);
    SANDY_HIP_TRY(hipModuleLoadData(&out->module, code.data()), e, "hipModuleLoadData");
    SANDY_HIP_TRY(hipModuleGetFunction(&out->fn, out->module, "sandy_ew"), e, "hipModuleGetFunction");
    return SANDY_OK;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

} // namespace

// exposed for the code-generation test entry below
std::string elementwise_source(const SandyScalarNode* nodes, int count, uint32_t result, const int32_t* in_dt,
                               const int* modes, int nin, int32_t out_dt, bool vec, int chunks_per_thread) {
    return generate(nodes, count, result, in_dt, modes, nin, out_dt, vec, chunks_per_thread);
}

} // namespace sandy_hip

using namespace sandy_hip;

extern "C" int sandy_hip_elementwise(const SandyScalarNode* nodes, int32_t node_count, uint32_t result,
                                     const SandyTensor* inputs, const int32_t* broadcast, int32_t input_count,
                                     const SandyTensor* out, void* stream_, char* err, size_t err_cap) {
    Err e{err, err_cap};
    hipStream_t stream = static_cast<hipStream_t>(stream_);
    if (input_count < 0 || input_count > SANDY_HIP_MAX_INPUTS)
        return fail(e, SANDY_ERR_INVALID, "elementwise input count exceeds kernel max inputs");
    if (node_count <= 0 || node_count > SANDY_HIP_MAX_SCALARS)
        return fail(e, SANDY_ERR_INVALID, "elementwise scalar count exceeds kernel max scalars");
    if (result >= SANDY_HIP_MAX_SCALARS) return fail(e, SANDY_ERR_INVALID, "elementwise result scalar id exceeds kernel max scalars");
    if (!valid_rank(out) || !is_float(out->dtype)) return fail(e, SANDY_ERR_INVALID, "elementwise output unsupported dtype");
    bool seen[SANDY_HIP_MAX_SCALARS] = {};
    for (int i = 0; i < node_count; i++) {
        const auto& n = nodes[i];
        if (n.id >= SANDY_HIP_MAX_SCALARS) return fail(e, SANDY_ERR_INVALID, "elementwise scalar id exceeds kernel max scalars");
        if (seen[n.id]) return fail(e, SANDY_ERR_INVALID, "elementwise duplicate scalar id");
        if (n.op < 0 || n.op > 15) return fail(e, SANDY_ERR_INVALID, "elementwise unknown scalar op");
        if (n.operand_count < 0 || n.operand_count > 2) return fail(e, SANDY_ERR_INVALID, "elementwise scalar op has too many operands");
        const int need = n.op == 0 || n.op == 1 ? 0 : (n.op >= 2 && n.op <= 7 ? 2 : 1);
        if (n.operand_count < need) return fail(e, SANDY_ERR_INVALID, "elementwise scalar op is missing operands");
        if (n.op == 0 && static_cast<int32_t>(n.input_index) >= input_count)
            return fail(e, SANDY_ERR_INVALID, "elementwise scalar load references invalid input");
        for (int j = 0; j < n.operand_count; j++) {
            if (n.operands[j] >= SANDY_HIP_MAX_SCALARS) return fail(e, SANDY_ERR_INVALID, "elementwise operand id exceeds kernel max scalars");
            if (!seen[n.operands[j]]) return fail(e, SANDY_ERR_INVALID, "elementwise scalar operands must be in dependency order");
        }
        seen[n.id] = true;
    }
    if (!seen[result]) return fail(e, SANDY_ERR_INVALID, "elementwise result references missing scalar");

    const int64_t n = numel(*out);
    EwArgs args{};
    int modes[SANDY_HIP_MAX_INPUTS] = {};
    int32_t dts[SANDY_HIP_MAX_INPUTS] = {};
    const bool out_contig = contiguous(*out);
    bool vec = out_contig && n % 8 == 0 && aligned16(base_ptr(*out));
    for (int i = 0; i < input_count; i++) {
        const SandyTensor& t = inputs[i];
        if (!valid_rank(&t) || !is_float(t.dtype)) return fail(e, SANDY_ERR_INVALID, "elementwise input unsupported dtype");
        const int64_t m = numel(t);
        dts[i] = t.dtype;
        args.in[i] = base_ptr(t);
        args.numel[i] = m;
        args.rank[i] = t.rank;
        for (int d = 0; d < t.rank; d++) {
            args.dims[i][d] = t.dims[d];
            args.strides[i][d] = t.strides[d];
        }
        const bool bc = broadcast && broadcast[i];
        if (!bc && m != n) return fail(e, SANDY_ERR_INVALID, "elementwise input shape mismatch");
        if (m == 1) modes[i] = kScalar;
        else if (!contiguous(t)) {
            if (bc) return fail(e, SANDY_ERR_UNSUPPORTED, "elementwise broadcast input must be contiguous");
            modes[i] = kStrided;
            vec = false;
        } else modes[i] = bc ? kBroadcast : kContig;
        if (modes[i] == kBroadcast && (m % 8 != 0 || !aligned16(args.in[i]))) vec = false;
        if (modes[i] == kContig && !aligned16(args.in[i])) vec = false;
    }
    if (n == 0) return ok(e);
    args.out = base_ptr(*out);
    args.n = n;
    args.orank = out->rank;
    for (int d = 0; d < out->rank; d++) {
        args.odims[d] = out->dims[d];
        args.ostrides[d] = out_contig ? 0 : out->strides[d];
    }
    if (out_contig) {  // contiguous output: flat index
        args.orank = 1;
        args.odims[0] = n;
        args.ostrides[0] = 1;
    }

    const int U = vec_chunks(n);
    const std::string src = generate(nodes, node_count, result, dts, modes, input_count, out->dtype, vec, U);
    int dev = 0;
    SANDY_HIP_TRY(hipGetDevice(&dev), e, "hipGetDevice");
    Compiled c;
    {
        std::lock_guard<std::mutex> lock(g_mu);
        auto key = std::make_pair(dev, src);
        auto it = g_cache.find(key);
        if (it == g_cache.end()) {
            int st = compile(src, &c, e);
            if (st) return st;
            g_cache.emplace(key, c);
        } else {
            c = it->second;
        }
    }
    // vectorised: 256 U chunks of 8 per workgroup per grid stride, at most
    // 4096 workgroups (16 per CU); scalar: one element per thread
    const int64_t threads = vec ? (n / 8 + U - 1) / U : n;
    int64_t blocks64 = (threads + 255) / 256;
    if (vec) blocks64 = std::min<int64_t>(blocks64, 4096);
    const unsigned blocks = static_cast<unsigned>(blocks64);
    EwVecArgs vargs{};
    if (vec) {
        for (int i = 0; i < input_count; i++) {
            vargs.in[i] = args.in[i];
            vargs.numel[i] = args.numel[i];
        }
        vargs.out = args.out;
        vargs.n = args.n;
    }
    void* params[] = {vec ? static_cast<void*>(&vargs) : static_cast<void*>(&args)};
    SANDY_HIP_TRY(hipModuleLaunchKernel(c.fn, blocks, 1, 1, 256, 1, 1, 0, stream, params, nullptr), e,
                  "elementwise launch");
    return ok(e);
}
