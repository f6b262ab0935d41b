// dispatch_driver.cpp -- runs KernelIR ops of every OpKind through the
// reference-side binding (HipKernelDispatch.cpp) against the recording stub
// of the C ABI (record_stub.cpp) and prints one JSON line per case: its name,
// whether hip_run_kernel succeeded, its error, and the C-ABI calls it made.
// Built and checked by tests/test_binding.py.
#include "HipKernelDispatch.h"

#include <cstdio>
#include <memory>
#include <string>
#include <vector>

extern std::vector<std::string> g_calls;
extern void* const kFailStream;

namespace kir = sandy::ir::kernel_ir;
using sandy::core::DType;
using sandy::core::Shape;
using sandy::core::TensorDesc;
using sandy::device::HipDeviceBufferView;

namespace {

void* const kStream = reinterpret_cast<void*>(0x57);

// A dense row-major view of `dims` at device address `addr`.
HipDeviceBufferView dense(uintptr_t addr, std::vector<int64_t> dims, DType dt = DType::F32, int64_t offset = 0) {
    HipDeviceBufferView b;
    b.data = reinterpret_cast<void*>(addr);
    b.view.desc = TensorDesc(Shape(dims), dt);
    b.view.strides.resize(dims.size());
    int64_t s = 1;
    for (int i = static_cast<int>(dims.size()) - 1; i >= 0; --i) {
        b.view.strides[static_cast<size_t>(i)] = s;
        s *= dims[static_cast<size_t>(i)];
    }
    b.view.storageOffset = offset;
    return b;
}

// A paged input as CudaDevice::run builds it: page table address, logical
// shape with default strides, grow dim, page size and count.
HipDeviceBufferView paged(uintptr_t table, std::vector<int64_t> dims, int64_t grow, int64_t pageSize,
                          int64_t pageCount, DType dt = DType::F32) {
    auto b = dense(table, std::move(dims), dt);
    b.paged = true;
    b.growDim = grow;
    b.pageSize = pageSize;
    b.pageCount = pageCount;
    return b;
}

std::string json_str(const std::string& s) {
    std::string o = "\"";
    for (char c : s) {
        if (c == '"' || c == '\\') o += '\\';
        o += c;
    }
    return o + "\"";
}

void run(const char* name, const kir::Op& op, std::vector<HipDeviceBufferView> in, std::vector<HipDeviceBufferView> out,
         void* stream = kStream) {
    g_calls.clear();
    auto r = sandy::device::hip_run_kernel(op, in, out, stream);
    std::printf("{\"case\":%s,\"ok\":%s,\"error\":%s,\"calls\":[", json_str(name).c_str(), r ? "true" : "false",
                json_str(r ? "" : r.error()).c_str());
    for (size_t i = 0; i < g_calls.size(); ++i) std::printf("%s%s", i ? "," : "", g_calls[i].c_str());
    std::printf("]}\n");
}

} // namespace

int main() {
    using BM = kir::BroadcastMode;
    using SO = kir::ScalarOp;
    kir::OpId id = 0;

    // ---------------------------------------------------------- boundary ops
    {
        kir::InputOp op(id++, kir::InputSource{kir::InputSourceKind::Argument, 0, ""}, 0);
        run("input", op, {}, {dense(0x100, {4})});
        kir::TensorTupleCreateOp tup(id++, std::vector<kir::ValueId>{0, 1}, 2);
        run("tensor_tuple_create", tup, {dense(0x100, {4}), dense(0x200, {4})}, {dense(0x300, {4})});
        kir::DeviceTransferOp xfer(id++, 0, 1, 0, 1);
        run("device_transfer", xfer, {dense(0x100, {4})}, {dense(0x200, {4})});
        kir::PagedAppendOp app(id++, 0, 1);
        run("paged_append", app, {paged(0x100, {2, 3, 4}, 1, 2, 2), dense(0x200, {2, 1, 4})}, {});
    }
    // ---------------------------------------------------------- layout
    {
        kir::LayoutTransformOp op(id++, kir::LayoutTransformKind::Transpose, 0, 1, {1, 0});
        auto x = dense(0x1000, {3, 4});
        x.view.strides = {1, 3};  // a transposed view of a [4, 3] buffer
        x.view.storageOffset = 2;
        run("layout_transpose", op, {x}, {dense(0x2000, {3, 4})});
        run("layout_paged", op, {paged(0x1000, {2, 3, 4}, 1, 2, 2)}, {dense(0x2000, {2, 3, 4})});
    }
    // ---------------------------------------------------------- element-wise
    {
        std::vector<kir::ScalarNode> nodes = {
            kir::ScalarNode{0, SO::Load, DType::F32, 0, 0.0, {}},
            kir::ScalarNode{1, SO::Load, DType::F32, 1, 0.0, {}},
            kir::ScalarNode{2, SO::Constant, DType::F32, 0, 0.5, {}},
            kir::ScalarNode{3, SO::Mul, DType::F32, 0, 0.0, {0, 2}},
            kir::ScalarNode{4, SO::Add, DType::F32, 0, 0.0, {3, 1}},
        };
        kir::ElementwiseKernelOp op(id++,
                                    std::vector<kir::ElementwiseInput>{{0, BM::None}, {1, BM::RightAligned}}, 2, 4,
                                    nodes);
        run("elementwise_dense", op, {dense(0x1000, {2, 3, 4}, DType::BF16), dense(0x2000, {4}, DType::BF16)},
            {dense(0x3000, {2, 3, 4}, DType::BF16)});
        // the reference's RunElementwiseReadsPagedTensorF32 operand: [2, T = 3, 4]
        // growing along dim 1 in pages of 2 rows
        run("elementwise_paged", op, {paged(0x1000, {2, 3, 4}, 1, 2, 2), dense(0x2000, {4})},
            {dense(0x3000, {2, 3, 4})});
        run("elementwise_paged_both", op, {paged(0x1000, {2, 3, 4}, 1, 2, 2), paged(0x2000, {2, 3, 4}, 1, 2, 2)},
            {dense(0x3000, {2, 3, 4})});
        run("elementwise_arity", op, {dense(0x1000, {2, 3, 4})}, {dense(0x3000, {2, 3, 4})});
        run("elementwise_paged_output", op, {dense(0x1000, {2, 3, 4}), dense(0x2000, {4})},
            {paged(0x3000, {2, 3, 4}, 1, 2, 2)});
        auto strided = paged(0x1000, {2, 3, 4}, 1, 2, 2);
        strided.view.strides = {1, 2, 6};
        run("elementwise_paged_noncontiguous", op, {strided, dense(0x2000, {4})}, {dense(0x3000, {2, 3, 4})});
        auto offset = paged(0x1000, {2, 3, 4}, 1, 2, 2);
        offset.view.storageOffset = 4;
        run("elementwise_paged_offset", op, {offset, dense(0x2000, {4})}, {dense(0x3000, {2, 3, 4})});
        run("elementwise_error", op, {dense(0x1000, {2, 3, 4}), dense(0x2000, {4})}, {dense(0x3000, {2, 3, 4})},
            kFailStream);
        std::vector<kir::ScalarNode> three = {kir::ScalarNode{0, SO::Load, DType::F32, 0, 0.0, {}},
                                              kir::ScalarNode{1, SO::Add, DType::F32, 0, 0.0, {0, 0, 0}}};
        kir::ElementwiseKernelOp bad(id++, std::vector<kir::ElementwiseInput>{{0, BM::None}}, 1, 1, three);
        run("elementwise_three_operands", bad, {dense(0x1000, {4})}, {dense(0x3000, {4})});
    }
    // ---------------------------------------------------------- reduction
    {
        kir::ReductionKernelOp op(id++, kir::ReduceOp::Sum, 0, 1, {1}, true);
        run("reduction_sum", op, {dense(0x1000, {4, 8})}, {dense(0x2000, {4, 1})});
        run("reduction_paged", op, {paged(0x1000, {4, 8}, 0, 4, 1)}, {dense(0x2000, {4, 1})});
        kir::ReductionKernelOp mx(id++, kir::ReduceOp::Max, 0, 1, {1}, true);
        run("reduction_max", mx, {dense(0x1000, {4, 8})}, {dense(0x2000, {4, 1})});
        kir::ReductionKernelOp two(id++, kir::ReduceOp::Sum, 0, 1, {0, 1}, true);
        run("reduction_two_axes", two, {dense(0x1000, {4, 8})}, {dense(0x2000, {1, 1})});
    }
    // ---------------------------------------------------------- linear / matmul
    {
        kir::LinearKernelOp lin(id++, 0, 1, 2, 3);
        run("linear_bias", lin, {dense(0x1000, {2, 8}), dense(0x2000, {16, 8}), dense(0x3000, {16})},
            {dense(0x4000, {2, 16})});
        run("linear_no_bias", lin, {dense(0x1000, {2, 8}), dense(0x2000, {16, 8})}, {dense(0x4000, {2, 16})});
        run("linear_paged", lin, {paged(0x1000, {2, 8}, 0, 2, 1), dense(0x2000, {16, 8}), dense(0x3000, {16})},
            {dense(0x4000, {2, 16})});
        kir::MatMulKernelOp mm(id++, 0, 1, 2, false, true);
        run("matmul", mm, {dense(0x1000, {2, 8}, DType::BF16), dense(0x2000, {16, 8}, DType::BF16)},
            {dense(0x4000, {2, 16}, DType::BF16)});
        kir::MatMulKernelOp mt(id++, 0, 1, 2, true, false);
        run("matmul_transpose_lhs", mt, {dense(0x1000, {8, 2}), dense(0x2000, {8, 16})}, {dense(0x4000, {2, 16})});
        run("matmul_paged", mm, {dense(0x1000, {2, 8}), paged(0x2000, {16, 8}, 0, 4, 4)}, {dense(0x4000, {2, 16})});
    }
    // ---------------------------------------------------------- gather / softmax / topk
    {
        kir::GatherKernelOp g(id++, 0, 1, 2);
        run("gather", g, {dense(0x1000, {5}, DType::I64), dense(0x2000, {100, 8})}, {dense(0x3000, {5, 8})});
        run("gather_paged_table", g, {dense(0x1000, {5}, DType::I32), paged(0x2000, {100, 8}, 0, 16, 7)},
            {dense(0x3000, {5, 8})});
        kir::SoftmaxKernelOp sm(id++, 0, 1, -1);
        run("softmax", sm, {dense(0x1000, {4, 8})}, {dense(0x2000, {4, 8})});
        run("softmax_paged", sm, {paged(0x1000, {2, 5, 8}, 1, 4, 2, DType::BF16)}, {dense(0x2000, {2, 5, 8}, DType::BF16)});
        run("softmax_error", sm, {dense(0x1000, {4, 8})}, {dense(0x2000, {4, 8})}, kFailStream);
        kir::TopKKernelOp tk(id++, 0, 1, 2, 8, -1);
        run("topk", tk, {dense(0x1000, {512, 128})}, {dense(0x2000, {512, 8}), dense(0x3000, {512, 8}, DType::I64)});
        run("topk_paged", tk, {paged(0x1000, {512, 128}, 0, 16, 32)},
            {dense(0x2000, {512, 8}), dense(0x3000, {512, 8}, DType::I64)});
        run("topk_arity", tk, {dense(0x1000, {512, 128})}, {dense(0x2000, {512, 8})});
    }
    // ---------------------------------------------------------- norm / rope
    {
        kir::NormKernelOp rms(id++, kir::NormKind::RMSNorm, std::vector<kir::ValueId>{0, 1}, 2, 1e-5);
        run("rms_norm", rms, {dense(0x1000, {4, 2048}, DType::BF16), dense(0x2000, {2048}, DType::BF16)},
            {dense(0x3000, {4, 2048}, DType::BF16)});
        kir::NormKernelOp rms0(id++, kir::NormKind::RMSNorm, std::vector<kir::ValueId>{0}, 1, 1e-6);
        run("rms_norm_no_weight", rms0, {dense(0x1000, {4, 64})}, {dense(0x3000, {4, 64})});
        kir::NormKernelOp ln(id++, kir::NormKind::LayerNorm, std::vector<kir::ValueId>{0, 1, 2}, 3, 1e-5);
        run("layer_norm", ln, {dense(0x1000, {4, 768}), dense(0x2000, {768}), dense(0x2800, {768})},
            {dense(0x3000, {4, 768})});
        run("rms_norm_paged", rms, {paged(0x1000, {1, 6, 64}, 1, 4, 2, DType::BF16), dense(0x2000, {64}, DType::BF16)},
            {dense(0x3000, {1, 6, 64}, DType::BF16)});
        kir::RoPEKernelOp rope(id++, 0, 1, 10000.0, -1, true);
        run("rope", rope, {dense(0x1000, {1, 32, 16, 64}, DType::BF16)}, {dense(0x2000, {1, 32, 16, 64}, DType::BF16)});
        kir::RoPEKernelOp ropeIds(id++, std::vector<kir::ValueId>{0, 1}, 2, 500000.0, 32, false);
        run("rope_ids", ropeIds, {dense(0x1000, {1, 8, 16, 64}), dense(0x1800, {16}, DType::I64)},
            {dense(0x2000, {1, 8, 16, 64})});
        run("rope_paged", ropeIds, {paged(0x1000, {1, 8, 16, 64}, 2, 16, 1), dense(0x1800, {16}, DType::I64)},
            {dense(0x2000, {1, 8, 16, 64})});
    }
    // ---------------------------------------------------------- attention
    {
        kir::AttentionKernelOp at(id++, 0, 1, 2, 3, 0, 0.125);
        run("attention_dense", at,
            {dense(0x1000, {1, 32, 4, 64}, DType::BF16), dense(0x2000, {1, 4, 4, 64}, DType::BF16),
             dense(0x3000, {1, 4, 4, 64}, DType::BF16)},
            {dense(0x4000, {1, 32, 4, 64}, DType::BF16)});
        kir::AttentionKernelOp ap(id++, 0, 1, 2, 3, 4, 128, -1.0);
        run("attention_paged_decode", ap,
            {dense(0x1000, {32, 32, 1, 64}, DType::BF16), paged(0x2000, {32, 4, 4096, 64}, 2, 16, 8192, DType::BF16),
             paged(0x3000, {32, 4, 4096, 64}, 2, 16, 8192, DType::BF16), dense(0x5000, {32}, DType::I64)},
            {dense(0x4000, {32, 32, 1, 64}, DType::BF16)});
        run("attention_paged_q", ap,
            {paged(0x1000, {2, 8, 1, 64}, 2, 1, 1, DType::BF16), paged(0x2000, {2, 4, 64, 64}, 2, 16, 8, DType::BF16),
             paged(0x3000, {2, 4, 64, 64}, 2, 16, 8, DType::BF16), dense(0x5000, {2}, DType::I32)},
            {dense(0x4000, {2, 8, 1, 64}, DType::BF16)});
        run("attention_paged_other_grow", ap,
            {dense(0x1000, {2, 8, 1, 64}), paged(0x2000, {2, 4, 64, 64}, 1, 2, 2), dense(0x3000, {2, 4, 64, 64}),
             dense(0x5000, {2}, DType::I64)},
            {dense(0x4000, {2, 8, 1, 64})});
        run("attention_arity", at, {dense(0x1000, {1, 32, 4, 64}), dense(0x2000, {1, 4, 4, 64})},
            {dense(0x4000, {1, 32, 4, 64})});
    }
    // ---------------------------------------------------------- MoE
    {
        kir::MoeGatherKernelOp g(id++, 0, 1, 2, 3, 4, 5, 6, 128, 8);
        std::vector<HipDeviceBufferView> outs = {dense(0x4000, {4096, 2816}, DType::BF16), dense(0x5000, {4096}, DType::BF16),
                                                 dense(0x6000, {4096}, DType::I64), dense(0x7000, {129}, DType::I64)};
        run("moe_gather", g,
            {dense(0x1000, {512, 2816}, DType::BF16), dense(0x2000, {512, 8}, DType::I64),
             dense(0x3000, {512, 8}, DType::BF16)},
            outs);
        run("moe_gather_paged_ids", g,
            {dense(0x1000, {512, 2816}, DType::BF16), paged(0x2000, {512, 8}, 0, 64, 8, DType::I64),
             dense(0x3000, {512, 8}, DType::BF16)},
            outs);
        kir::MoeMatMulKernelOp mm(id++, 0, 1, 2, 3, true);
        run("moe_matmul", mm,
            {dense(0x1000, {4096, 2816}, DType::BF16), dense(0x2000, {129}, DType::I64),
             dense(0x3000, {128, 704, 2816}, DType::BF16)},
            {dense(0x4000, {4096, 704}, DType::BF16)});
        run("moe_matmul_paged", mm,
            {paged(0x1000, {4096, 2816}, 0, 64, 64, DType::BF16), dense(0x2000, {129}, DType::I64),
             dense(0x3000, {128, 704, 2816}, DType::BF16)},
            {dense(0x4000, {4096, 704}, DType::BF16)});
        kir::MoeScatterSumKernelOp ss(id++, 0, 1, 2, 3, 4);
        run("moe_scatter_sum", ss,
            {dense(0x1000, {4096, 2816}, DType::BF16), dense(0x2000, {4096}, DType::BF16),
             dense(0x3000, {4096}, DType::I64), dense(0x3800, {512, 2816}, DType::BF16)},
            {dense(0x4000, {512, 2816}, DType::BF16)});
        run("moe_scatter_sum_paged_tokens", ss,
            {dense(0x1000, {4096, 2816}, DType::BF16), dense(0x2000, {4096}, DType::BF16),
             paged(0x3000, {4096}, 0, 64, 64, DType::I64), dense(0x3800, {512, 2816}, DType::BF16)},
            {dense(0x4000, {512, 2816}, DType::BF16)});
    }
    // ---------------------------------------------------------- not part of this backend
    {
        kir::SlidingQueryKeyScoreKernelOp op(id++, 0, 1, 2, 64, 0.125);
        run("sliding_query_key_score", op, {dense(0x1000, {1, 4, 8, 64}), dense(0x2000, {1, 4, 8, 64})},
            {dense(0x3000, {1, 4, 8, 8})});
    }
    return 0;
}
