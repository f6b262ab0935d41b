// gpu_driver.cpp -- runs KernelIR ops through the reference-side binding
// (HipKernelDispatch.cpp) against the real libsandyrt_hip on the GPU: the ops
// are the reference's own kir::Op classes (src/ir/KernelIR.h), the operands
// device buffers of the library's Device API, paged operands the reference's
// page-address layout (CudaPagedTensor.cpp:187-226).  One JSON line per case:
// its name, whether hip_run_kernel succeeded, its error, and every input and
// output tensor (bf16 as raw 16-bit words), which tests/test_gpu_binding.py
// checks against the CPU oracle.  Built by oracle/Makefile (target
// binding) from the reference sources where they exist; run on the GPU.
#include "HipKernelDispatch.h"

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

namespace kir = sandy::ir::kernel_ir;
using sandy::core::DType;
using sandy::core::Shape;
using sandy::core::TensorDesc;
using sandy::device::HipDeviceBufferView;

namespace {

SandyHipDevice* g_dev = nullptr;
char g_err[512];

void die(const char* what) {
    std::fprintf(stderr, "%s: %s\n", what, g_err);
    std::exit(2);
}

// Deterministic inputs: a 64-bit LCG mapped to [-1, 1).
struct Lcg {
    uint64_t s;
    explicit Lcg(uint64_t seed) : s(seed * 6364136223846793005ull + 1442695040888963407ull) {}
    float next() {
        s = s * 6364136223846793005ull + 1442695040888963407ull;
        return static_cast<float>(static_cast<int64_t>(s >> 40) - (1 << 23)) / static_cast<float>(1 << 23);
    }
};

uint16_t to_bf16(float f) {  // round to nearest even (src/core/Tensor.h:43-49)
    uint32_t b;
    std::memcpy(&b, &f, 4);
    return static_cast<uint16_t>((b + 0x7fffu + ((b >> 16) & 1u)) >> 16);
}

// A host tensor: raw bytes, dtype and shape, and the device buffer it lives in.
struct HostTensor {
    std::string name;
    DType dt;
    std::vector<int64_t> dims;
    std::vector<unsigned char> bytes;
    uint32_t buffer = 0;
    int64_t numel() const {
        int64_t n = 1;
        for (int64_t d : dims) n *= d;
        return n;
    }
};

size_t elem_size(DType dt) { return dt == DType::BF16 ? 2 : dt == DType::I64 ? 8 : 4; }

HostTensor random_tensor(const char* name, DType dt, std::vector<int64_t> dims, uint64_t seed, float scale = 1.0f) {
    HostTensor t{name, dt, std::move(dims), {}};
    const int64_t n = t.numel();
    t.bytes.resize(static_cast<size_t>(n) * elem_size(dt));
    Lcg r(seed);
    for (int64_t i = 0; i < n; ++i) {
        const float v = r.next() * scale;
        if (dt == DType::BF16) {
            const uint16_t h = to_bf16(v);
            std::memcpy(&t.bytes[static_cast<size_t>(i) * 2], &h, 2);
        } else {
            std::memcpy(&t.bytes[static_cast<size_t>(i) * 4], &v, 4);
        }
    }
    return t;
}

template <typename I>
HostTensor index_tensor(const char* name, DType dt, std::vector<int64_t> dims, const std::vector<I>& values) {
    HostTensor t{name, dt, std::move(dims), {}};
    t.bytes.resize(values.size() * sizeof(I));
    std::memcpy(t.bytes.data(), values.data(), t.bytes.size());
    return t;
}

HostTensor empty_tensor(const char* name, DType dt, std::vector<int64_t> dims) {
    HostTensor t{name, dt, std::move(dims), {}};
    t.bytes.assign(static_cast<size_t>(t.numel()) * elem_size(dt), 0);
    return t;
}

void upload(HostTensor& t) {
    if (sandy_hip_device_load(g_dev, t.bytes.data(), t.bytes.size(), &t.buffer, g_err, sizeof g_err)) die("load");
}

void download(HostTensor& t) {
    if (sandy_hip_device_read(g_dev, t.buffer, 0, t.bytes.size(), t.bytes.data(), g_err, sizeof g_err)) die("read");
}

HipDeviceBufferView dense_view(const HostTensor& t) {
    HipDeviceBufferView b;
    b.data = sandy_hip_device_buffer(g_dev, t.buffer);
    b.view.desc = TensorDesc(Shape(t.dims), t.dt);
    b.view.strides.resize(t.dims.size());
    int64_t s = 1;
    for (int i = static_cast<int>(t.dims.size()) - 1; i >= 0; --i) {
        b.view.strides[static_cast<size_t>(i)] = s;
        s *= t.dims[static_cast<size_t>(i)];
    }
    return b;
}

// The reference's paged layout of a logical tensor t growing along `grow`:
// page p holds [prefix dims, page_size, inner dims] for grow rows
// [p * page_size, (p + 1) * page_size), each page its own allocation, and the
// operand's data is the device array of page start addresses.
struct PagedOperand {
    std::vector<HostTensor> pages;
    HostTensor table;
    HipDeviceBufferView view;
};

PagedOperand make_paged(const HostTensor& t, int grow, int64_t page_size) {
    PagedOperand p;
    const size_t es = elem_size(t.dt);
    int64_t prefix = 1, inner = 1;
    for (int i = 0; i < grow; ++i) prefix *= t.dims[static_cast<size_t>(i)];
    for (size_t i = static_cast<size_t>(grow) + 1; i < t.dims.size(); ++i) inner *= t.dims[i];
    const int64_t len = t.dims[static_cast<size_t>(grow)];
    const int64_t count = (len + page_size - 1) / page_size;
    std::vector<uint64_t> addrs;
    for (int64_t pg = 0; pg < count; ++pg) {
        HostTensor page = empty_tensor("page", t.dt, {prefix, page_size, inner});
        for (int64_t a = 0; a < prefix; ++a)
            for (int64_t r = 0; r < page_size; ++r) {
                const int64_t row = pg * page_size + r;
                if (row >= len) continue;
                std::memcpy(&page.bytes[static_cast<size_t>((a * page_size + r) * inner) * es],
                            &t.bytes[static_cast<size_t>((a * len + row) * inner) * es], static_cast<size_t>(inner) * es);
            }
        upload(page);
        addrs.push_back(reinterpret_cast<uint64_t>(sandy_hip_device_buffer(g_dev, page.buffer)));
        p.pages.push_back(std::move(page));
    }
    p.table = index_tensor("table", DType::I64, {count}, addrs);
    upload(p.table);
    p.view = dense_view(t);
    p.view.data = sandy_hip_device_buffer(g_dev, p.table.buffer);
    p.view.paged = true;
    p.view.growDim = grow;
    p.view.pageSize = page_size;
    p.view.pageCount = count;
    return p;
}

const char* short_dtype(DType dt) {
    switch (dt) {
    case DType::BF16: return "bf16";
    case DType::F32: return "f32";
    case DType::I32: return "i32";
    case DType::I64: return "i64";
    default: return "?";
    }
}

void print_tensor(const HostTensor& t, bool first) {
    std::printf("%s\"%s\":{\"dtype\":\"%s\",\"shape\":[", first ? "" : ",", t.name.c_str(), short_dtype(t.dt));
    for (size_t i = 0; i < t.dims.size(); ++i) std::printf("%s%lld", i ? "," : "", static_cast<long long>(t.dims[i]));
    std::printf("],\"data\":[");
    const int64_t n = t.numel();
    for (int64_t i = 0; i < n; ++i) {
        const unsigned char* p = &t.bytes[static_cast<size_t>(i) * elem_size(t.dt)];
        if (i) std::printf(",");
        if (t.dt == DType::BF16) {
            uint16_t v;
            std::memcpy(&v, p, 2);
            std::printf("%u", v);
        } else if (t.dt == DType::F32) {
            float v;
            std::memcpy(&v, p, 4);
            std::printf("%.9g", v);
        } else if (t.dt == DType::I32) {
            int32_t v;
            std::memcpy(&v, p, 4);
            std::printf("%d", v);
        } else {
            int64_t v;
            std::memcpy(&v, p, 8);
            std::printf("%lld", static_cast<long long>(v));
        }
    }
    std::printf("]}");
}

std::string json_str(const std::string& s) {
    std::string o = "\"";
    for (char c : s) {
        if (c == '"' || c == '\\') o += '\\';
        o += c;
    }
    return o + "\"";
}

// Runs `op` on the device's stream, reads every output back and prints the case.
void run(const char* name, const kir::Op& op, std::vector<HipDeviceBufferView> in, std::vector<HostTensor*> inputs,
         std::vector<HostTensor*> outputs) {
    std::vector<HipDeviceBufferView> out;
    for (HostTensor* t : outputs) {
        upload(*t);  // zero-filled
        out.push_back(dense_view(*t));
    }
    std::fprintf(stderr, "case %s\n", name);
    std::fflush(stderr);
    auto r = sandy::device::hip_run_kernel(op, in, out, sandy_hip_device_stream(g_dev));
    std::string error = r ? "" : r.error();
    if (r) {
        uint32_t flags = 0;
        if (sandy_hip_take_device_errors(sandy_hip_device_stream(g_dev), &flags, g_err, sizeof g_err)) error = g_err;
        for (HostTensor* t : outputs) download(*t);
    }
    std::printf("{\"case\":%s,\"ok\":%s,\"error\":%s,\"tensors\":{", json_str(name).c_str(),
                error.empty() ? "true" : "false", json_str(error).c_str());
    bool first = true;
    for (HostTensor* t : inputs) {
        print_tensor(*t, first);
        first = false;
    }
    for (HostTensor* t : outputs) {
        print_tensor(*t, first);
        first = false;
    }
    std::printf("}}\n");
    std::fflush(stdout);
}

} // namespace

int main() {
    using BM = kir::BroadcastMode;
    using SO = kir::ScalarOp;
    if (sandy_hip_device_create(0, &g_dev, g_err, sizeof g_err)) die("device");
    kir::OpId id = 0;

    // element-wise group 0.5 * x + y, y broadcast along the last dim, bf16
    std::vector<kir::ScalarNode> nodes = {
        kir::ScalarNode{0, SO::Load, DType::F32, 0, 0.0, {}},
        kir::ScalarNode{1, SO::Load, DType::F32, 1, 0.0, {}},
        kir::ScalarNode{2, SO::Constant, DType::F32, 0, 0.5, {}},
        kir::ScalarNode{3, SO::Mul, DType::F32, 0, 0.0, {0, 2}},
        kir::ScalarNode{4, SO::Add, DType::F32, 0, 0.0, {3, 1}},
    };
    kir::ElementwiseKernelOp ew(id++, std::vector<kir::ElementwiseInput>{{0, BM::None}, {1, BM::RightAligned}}, 2, 4,
                                nodes);
    {
        HostTensor x = random_tensor("x", DType::BF16, {2, 3, 64}, 1), y = random_tensor("y", DType::BF16, {64}, 2);
        HostTensor o = empty_tensor("out", DType::BF16, {2, 3, 64});
        upload(x);
        upload(y);
        run("elementwise_bf16", ew, {dense_view(x), dense_view(y)}, {&x, &y}, {&o});
    }
    // the same group over a paged f32 input [2, T = 5, 8] in pages of 2 rows
    {
        HostTensor x = random_tensor("x", DType::F32, {2, 5, 8}, 3), y = random_tensor("y", DType::F32, {8}, 4);
        HostTensor o = empty_tensor("out", DType::F32, {2, 5, 8});
        PagedOperand px = make_paged(x, 1, 2);
        upload(y);
        run("elementwise_paged_f32", ew, {px.view, dense_view(y)}, {&x, &y}, {&o});
    }
    // RMSNorm with weight, bf16 [4, 2048]
    {
        kir::NormKernelOp rms(id++, kir::NormKind::RMSNorm, std::vector<kir::ValueId>{0, 1}, 2, 1e-5);
        HostTensor x = random_tensor("x", DType::BF16, {4, 2048}, 5), w = random_tensor("w", DType::BF16, {2048}, 6);
        HostTensor o = empty_tensor("out", DType::BF16, {4, 2048});
        upload(x);
        upload(w);
        run("rms_norm_bf16", rms, {dense_view(x), dense_view(w)}, {&x, &w}, {&o});
    }
    // split-half RoPE, theta 1e4, bf16 [1, 4, 16, 64]
    {
        kir::RoPEKernelOp rope(id++, 0, 1, 10000.0, -1, true);
        HostTensor x = random_tensor("x", DType::BF16, {1, 4, 16, 64}, 7);
        HostTensor o = empty_tensor("out", DType::BF16, {1, 4, 16, 64});
        upload(x);
        run("rope_bf16", rope, {dense_view(x)}, {&x}, {&o});
    }
    // softmax over the last dim, f32 [4, 33]
    {
        kir::SoftmaxKernelOp sm(id++, 0, 1, -1);
        HostTensor x = random_tensor("x", DType::F32, {4, 33}, 8, 4.0f);
        HostTensor o = empty_tensor("out", DType::F32, {4, 33});
        upload(x);
        run("softmax_f32", sm, {dense_view(x)}, {&x}, {&o});
    }
    // top-8 of 128, f32 [8, 128], int64 indices
    {
        kir::TopKKernelOp tk(id++, 0, 1, 2, 8, -1);
        HostTensor x = random_tensor("x", DType::F32, {8, 128}, 9);
        HostTensor v = empty_tensor("values", DType::F32, {8, 8}), i = empty_tensor("indices", DType::I64, {8, 8});
        upload(x);
        run("topk_f32", tk, {dense_view(x)}, {&x}, {&v, &i});
    }
    // paged decode attention: q [2, 8, 1, 64] bf16, K/V [2, 2, 64, 64] in the
    // reference's paged layout (grow dim 2, pages of 16 keys), positions 37 and 63
    {
        kir::AttentionKernelOp at(id++, 0, 1, 2, 3, 4, 0, -1.0);
        HostTensor q = random_tensor("q", DType::BF16, {2, 8, 1, 64}, 10);
        HostTensor k = random_tensor("k", DType::BF16, {2, 2, 64, 64}, 11);
        HostTensor v = random_tensor("v", DType::BF16, {2, 2, 64, 64}, 12);
        HostTensor pos = index_tensor("pos", DType::I64, {2}, std::vector<int64_t>{37, 63});
        HostTensor o = empty_tensor("out", DType::BF16, {2, 8, 1, 64});
        upload(q);
        upload(pos);
        PagedOperand pk = make_paged(k, 2, 16), pv = make_paged(v, 2, 16);
        run("attention_paged_decode_bf16", at, {dense_view(q), pk.view, pv.view, dense_view(pos)}, {&q, &k, &v, &pos},
            {&o});
    }
    // MoE: gather (8 tokens, top-2 of 4 experts) -> grouped GEMM [4, 32, 64] -> scatter-sum
    {
        const int64_t T = 8, K = 2, E = 4, H = 64, F = 32;
        HostTensor x = random_tensor("x", DType::BF16, {T, H}, 13);
        std::vector<int64_t> ids = {0, 1, 2, 3, 1, 2, 3, 0, 0, 2, 1, 3, 2, 0, 3, 1};
        HostTensor tid = index_tensor("topk_ids", DType::I64, {T, K}, ids);
        HostTensor tw = random_tensor("topk_weights", DType::BF16, {T, K}, 14);
        HostTensor w = random_tensor("weight", DType::BF16, {E, F, H}, 15);
        HostTensor px = empty_tensor("packed_x", DType::BF16, {T * K, H});
        HostTensor pw = empty_tensor("packed_w", DType::BF16, {T * K});
        HostTensor tok = empty_tensor("token_ids", DType::I64, {T * K});
        HostTensor off = empty_tensor("offsets", DType::I64, {E + 1});
        upload(x);
        upload(tid);
        upload(tw);
        upload(w);
        kir::MoeGatherKernelOp g(id++, 0, 1, 2, 3, 4, 5, 6, E, K);
        run("moe_gather_bf16", g, {dense_view(x), dense_view(tid), dense_view(tw)}, {&x, &tid, &tw},
            {&px, &pw, &tok, &off});
        HostTensor mo = empty_tensor("packed_out", DType::BF16, {T * K, F});
        kir::MoeMatMulKernelOp mm(id++, 0, 1, 2, 3, true);
        run("moe_matmul_bf16", mm, {dense_view(px), dense_view(off), dense_view(w)}, {&px, &off, &w}, {&mo});
        HostTensor ref = empty_tensor("reference", DType::BF16, {T, F});
        upload(ref);
        HostTensor so = empty_tensor("out", DType::BF16, {T, F});
        kir::MoeScatterSumKernelOp ss(id++, 0, 1, 2, 3, 4);
        run("moe_scatter_sum_bf16", ss, {dense_view(mo), dense_view(pw), dense_view(tok), dense_view(ref)},
            {&mo, &pw, &tok}, {&so});
    }
    // reduction: sum over the last dim, keep dims, f32 [4, 300]
    {
        kir::ReductionKernelOp op(id++, kir::ReduceOp::Sum, 0, 1, {1}, true);
        HostTensor x = random_tensor("x", DType::F32, {4, 300}, 16);
        HostTensor o = empty_tensor("out", DType::F32, {4, 1});
        upload(x);
        run("reduce_sum_f32", op, {dense_view(x)}, {&x}, {&o});
    }
    // linear with bias, f32 [3, 96] x [40, 96]^T + [40]
    {
        kir::LinearKernelOp op(id++, 0, 1, 2, 3);
        HostTensor x = random_tensor("x", DType::F32, {3, 96}, 17), w = random_tensor("w", DType::F32, {40, 96}, 18);
        HostTensor b = random_tensor("b", DType::F32, {40}, 19);
        HostTensor o = empty_tensor("out", DType::F32, {3, 40});
        upload(x);
        upload(w);
        upload(b);
        run("linear_f32", op, {dense_view(x), dense_view(w), dense_view(b)}, {&x, &w, &b}, {&o});
    }
    // matmul, rhs transposed, bf16 [2, 5, 128] x [2, 48, 128]^T
    {
        kir::MatMulKernelOp op(id++, 0, 1, 2, false, true);
        HostTensor l = random_tensor("lhs", DType::BF16, {2, 5, 128}, 20);
        HostTensor r = random_tensor("rhs", DType::BF16, {2, 48, 128}, 21);
        HostTensor o = empty_tensor("out", DType::BF16, {2, 5, 48});
        upload(l);
        upload(r);
        run("matmul_bf16", op, {dense_view(l), dense_view(r)}, {&l, &r}, {&o});
    }
    // gather (embedding rows), int64 ids into a bf16 [50, 64] table
    {
        kir::GatherKernelOp op(id++, 0, 1, 2);
        HostTensor ids = index_tensor("ids", DType::I64, {6}, std::vector<int64_t>{3, 0, 49, 3, 17, 8});
        HostTensor t = random_tensor("table", DType::BF16, {50, 64}, 22);
        HostTensor o = empty_tensor("out", DType::BF16, {6, 64});
        upload(ids);
        upload(t);
        run("gather_bf16", op, {dense_view(ids), dense_view(t)}, {&ids, &t}, {&o});
    }
    // LayerNorm with weight and bias, f32 [3, 768]
    {
        kir::NormKernelOp ln(id++, kir::NormKind::LayerNorm, std::vector<kir::ValueId>{0, 1, 2}, 3, 1e-5);
        HostTensor x = random_tensor("x", DType::F32, {3, 768}, 23), w = random_tensor("w", DType::F32, {768}, 24);
        HostTensor b = random_tensor("b", DType::F32, {768}, 25);
        HostTensor o = empty_tensor("out", DType::F32, {3, 768});
        upload(x);
        upload(w);
        upload(b);
        run("layer_norm_f32", ln, {dense_view(x), dense_view(w), dense_view(b)}, {&x, &w, &b}, {&o});
    }
    // interleaved partial RoPE with position ids, theta 5e5, f32 [1, 2, 16, 64]
    {
        kir::RoPEKernelOp rope(id++, std::vector<kir::ValueId>{0, 1}, 2, 500000.0, 32, false);
        HostTensor x = random_tensor("x", DType::F32, {1, 2, 16, 64}, 26);
        std::vector<int64_t> p(16);
        for (int i = 0; i < 16; ++i) p[static_cast<size_t>(i)] = 1000 + 37 * i;
        HostTensor ids = index_tensor("ids", DType::I64, {16}, p);
        HostTensor o = empty_tensor("out", DType::F32, {1, 2, 16, 64});
        upload(x);
        upload(ids);
        run("rope_ids_f32", rope, {dense_view(x), dense_view(ids)}, {&x, &ids}, {&o});
    }
    // layout: a transposed view of a [4, 6] f32 buffer made contiguous
    {
        kir::LayoutTransformOp op(id++, kir::LayoutTransformKind::Transpose, 0, 1, {1, 0});
        HostTensor x = random_tensor("x", DType::F32, {4, 6}, 27);
        HostTensor o = empty_tensor("out", DType::F32, {6, 4});
        upload(x);
        HipDeviceBufferView v = dense_view(x);
        v.view.desc = TensorDesc(Shape(std::vector<int64_t>{6, 4}), DType::F32);
        v.view.strides = {1, 6};
        run("layout_transpose_f32", op, {v}, {&x}, {&o});
    }
    // softmax over a paged bf16 input [2, 5, 8] (grow dim 1, pages of 4 rows)
    {
        kir::SoftmaxKernelOp sm(id++, 0, 1, -1);
        HostTensor x = random_tensor("x", DType::BF16, {2, 5, 8}, 28, 3.0f);
        HostTensor o = empty_tensor("out", DType::BF16, {2, 5, 8});
        PagedOperand px = make_paged(x, 1, 4);
        run("softmax_paged_bf16", sm, {px.view}, {&x}, {&o});
    }
    // dense attention (prefill, causal from positions), bf16 q [1, 8, 4, 64], K/V [1, 2, 12, 64]
    {
        kir::AttentionKernelOp at(id++, 0, 1, 2, 3, 4, 0, -1.0);
        HostTensor q = random_tensor("q", DType::BF16, {1, 8, 4, 64}, 29);
        HostTensor k = random_tensor("k", DType::BF16, {1, 2, 12, 64}, 30);
        HostTensor v = random_tensor("v", DType::BF16, {1, 2, 12, 64}, 31);
        HostTensor pos = index_tensor("pos", DType::I64, {1}, std::vector<int64_t>{8});
        HostTensor o = empty_tensor("out", DType::BF16, {1, 8, 4, 64});
        upload(q);
        upload(k);
        upload(v);
        upload(pos);
        run("attention_dense_bf16", at, {dense_view(q), dense_view(k), dense_view(v), dense_view(pos)},
            {&q, &k, &v, &pos}, {&o});
    }
    sandy_hip_device_destroy(g_dev);
    return 0;
}
