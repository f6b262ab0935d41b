// HipKernelDispatch.cpp -- the reference-side binding of libsandyrt_hip.
//
// A SandyRT maintainer adds this file to the reference tree as
// src/device/hip/HipKernelDispatch.cpp.  It is the dispatch a HipDevice::run
// performs once it has resolved its DeviceRunValues to buffer views: the
// place where CudaDevice::run calls launch_cuda_<family>
// (src/device/cuda/CudaDevice.cpp:520-578).  Each KernelIR op is converted
// field for field into the plain descriptors of include/sandyrt_hip.h and
// handed to one sandy_hip_* entry point; the status and message come back as
// the reference's Result<void>.  It depends only on the reference's own
// headers (KernelIR.h, DeviceTypes.h, Result.h, Tensor.h) and sandyrt_hip.h;
// tests/test_binding.py compiles it against them.
#include "DeviceTypes.h"
#include "KernelIR.h"
#include "Result.h"
#include "Tensor.h"
#include "sandyrt_hip.h"

#include <cstdint>
#include <span>
#include <string>
#include <vector>

namespace sandy::device {

// One operand of a launch, as HipDevice::run resolves it -- the fields of
// CudaDeviceBufferView (src/device/cuda/CudaKernels.h:19-28).  Dense: `data`
// is the allocation's device address and `view` its strides and storage
// offset.  Paged (the reference's CudaPagedTensor layout): `data` is the
// device array of page start addresses, `view.desc` the logical shape, and
// growDim / pageSize / pageCount describe the pages.
struct HipDeviceBufferView {
    void* data = nullptr;
    TensorViewDesc view;
    bool paged = false;
    int64_t growDim = -1;
    int64_t pageSize = -1;
    int64_t pageCount = 0;
};

namespace {

namespace kir = ir::kernel_ir;

SandyTensor to_tensor(const HipDeviceBufferView& b) {
    SandyTensor t{};
    t.data = b.data;
    t.dtype = static_cast<int32_t>(b.view.desc.dtype);  // SandyDType follows core::DType (Tensor.h:13)
    t.rank = b.view.desc.shape.rank();
    for (int i = 0; i < t.rank && i < SANDY_HIP_MAX_RANK; ++i) {
        t.dims[i] = b.view.desc.shape.dim(i);
        t.strides[i] = i < static_cast<int>(b.view.strides.size()) ? b.view.strides[i] : 0;
    }
    t.storage_offset = b.view.storageOffset;
    return t;
}

SandyPagedView to_paged(const HipDeviceBufferView& b) {
    SandyPagedView p{};
    p.pages = b.data;
    p.dtype = static_cast<int32_t>(b.view.desc.dtype);
    p.rank = b.view.desc.shape.rank();
    for (int i = 0; i < p.rank && i < 4; ++i) p.dims[i] = b.view.desc.shape.dim(i);
    p.page_size = b.pageSize;
    p.page_count = b.pageCount;
    return p;
}

// The call's status as the reference's Result: the message is already worded
// like the reference's errors.
Result<void> result(int rc, const char* err) {
    if (rc == SANDY_OK) return {};
    return make_error(std::string(err));
}

Result<void> dense_only(std::span<const HipDeviceBufferView> views, const char* kernel) {
    for (const auto& v : views)
        if (v.paged) return make_error(std::string("hip ") + kernel + " does not support paged tensors");
    return {};
}

Result<void> arity(std::span<const HipDeviceBufferView> in, std::span<const HipDeviceBufferView> out, size_t minIn,
                   size_t minOut, const char* kernel) {
    if (in.size() < minIn) return make_error(std::string("hip ") + kernel + " input arity mismatch");
    if (out.size() < minOut) return make_error(std::string("hip ") + kernel + " output arity mismatch");
    return {};
}

} // namespace

// Runs one KernelIR op on `stream` (a hipStream_t).  `inputs` / `outputs`
// follow the op's inputs() / outputs() order, as CudaDevice::run builds its
// CudaLaunchContext.
Result<void> hip_run_kernel(const kir::Op& op, std::span<const HipDeviceBufferView> inputs,
                            std::span<const HipDeviceBufferView> outputs, void* stream) {
    char err[512] = {0};
    auto in = [&](size_t i) { return to_tensor(inputs[i]); };
    auto out = [&](size_t i) { return to_tensor(outputs[i]); };

    switch (op.kind()) {
        case kir::OpKind::Input:
        case kir::OpKind::TensorTupleCreate:
        case kir::OpKind::DeviceTransfer:
        case kir::OpKind::PagedAppend:
            return make_error("hip device cannot run boundary op");

        case kir::OpKind::LayoutTransform: {
            const auto& k = static_cast<const kir::LayoutTransformOp&>(op);
            if (auto a = arity(inputs, outputs, 1, 1, "layout_transform"); !a) return a;
            if (auto d = dense_only(inputs, "layout_transform"); !d) return d;
            auto x = in(0), y = out(0);
            return result(sandy_hip_layout_transform(&x, &y, static_cast<int32_t>(k.transform()), stream, err,
                                                     sizeof err),
                          err);
        }

        case kir::OpKind::ElementwiseKernel: {
            const auto& k = static_cast<const kir::ElementwiseKernelOp&>(op);
            if (auto a = arity(inputs, outputs, k.elementwiseInputs().size(), 1, "elementwise"); !a) return a;
            if (auto d = dense_only(inputs, "elementwise"); !d) return d;
            std::vector<SandyScalarNode> nodes;
            nodes.reserve(k.scalars().size());
            for (const auto& s : k.scalars()) {
                if (s.operands.size() > 2) return make_error("hip elementwise scalar node has more than two operands");
                SandyScalarNode n{};
                n.id = s.id;
                n.op = static_cast<int32_t>(s.op);  // ScalarOp order, KernelIR.h:317-337
                n.dtype = static_cast<int32_t>(s.dtype);
                n.input_index = s.inputIndex;
                n.constant = s.constant;
                n.operand_count = static_cast<int32_t>(s.operands.size());
                for (size_t j = 0; j < s.operands.size(); ++j) n.operands[j] = s.operands[j];
                nodes.push_back(n);
            }
            std::vector<SandyTensor> xs;
            std::vector<int32_t> bc;
            for (size_t i = 0; i < k.elementwiseInputs().size(); ++i) {
                xs.push_back(in(i));
                bc.push_back(k.elementwiseInputs()[i].broadcast == kir::BroadcastMode::RightAligned ? 1 : 0);
            }
            auto y = out(0);
            return result(sandy_hip_elementwise(nodes.data(), static_cast<int32_t>(nodes.size()), k.result(),
                                                xs.data(), bc.data(), static_cast<int32_t>(xs.size()), &y, stream,
                                                err, sizeof err),
                          err);
        }

        case kir::OpKind::ReductionKernel: {
            const auto& k = static_cast<const kir::ReductionKernelOp&>(op);
            if (auto a = arity(inputs, outputs, 1, 1, "reduction"); !a) return a;
            if (k.reduce() != kir::ReduceOp::Sum) return make_error("hip reduction only supports sum");
            if (k.axes().size() != 1) return make_error("hip reduction only supports one axis");
            auto x = in(0), y = out(0);
            return result(sandy_hip_reduce_sum(&x, k.axes()[0], k.keepDims() ? 1 : 0, &y, stream, err, sizeof err),
                          err);
        }

        case kir::OpKind::LinearKernel: {
            if (auto a = arity(inputs, outputs, 2, 1, "linear"); !a) return a;
            auto x = in(0), w = in(1), y = out(0);
            SandyTensor b{};
            const bool hasBias = inputs.size() > 2;
            if (hasBias) b = in(2);
            return result(sandy_hip_linear(&x, &w, hasBias ? &b : nullptr, &y, stream, err, sizeof err), err);
        }

        case kir::OpKind::MatMulKernel: {
            const auto& k = static_cast<const kir::MatMulKernelOp&>(op);
            if (auto a = arity(inputs, outputs, 2, 1, "matmul"); !a) return a;
            if (auto d = dense_only(inputs, "matmul"); !d) return d;
            auto lhs = in(0), rhs = in(1), y = out(0);
            return result(sandy_hip_matmul(&lhs, &rhs, k.transposeLhs() ? 1 : 0, k.transposeRhs() ? 1 : 0, &y, stream,
                                           err, sizeof err),
                          err);
        }

        case kir::OpKind::GatherKernel: {
            if (auto a = arity(inputs, outputs, 2, 1, "gather"); !a) return a;
            auto ids = in(0), table = in(1), y = out(0);
            return result(sandy_hip_gather(&ids, &table, &y, stream, err, sizeof err), err);
        }

        case kir::OpKind::SoftmaxKernel: {
            const auto& k = static_cast<const kir::SoftmaxKernelOp&>(op);
            if (auto a = arity(inputs, outputs, 1, 1, "softmax"); !a) return a;
            auto x = in(0), y = out(0);
            return result(sandy_hip_softmax(&x, k.axis(), &y, stream, err, sizeof err), err);
        }

        case kir::OpKind::TopKKernel: {
            const auto& k = static_cast<const kir::TopKKernelOp&>(op);
            if (auto a = arity(inputs, outputs, 1, 2, "topk"); !a) return a;
            auto x = in(0), values = out(0), indices = out(1);
            return result(sandy_hip_topk(&x, k.k(), k.axis(), &values, &indices, stream, err, sizeof err), err);
        }

        case kir::OpKind::NormKernel: {
            const auto& k = static_cast<const kir::NormKernelOp&>(op);
            if (auto a = arity(inputs, outputs, 1, 1, "norm"); !a) return a;
            auto x = in(0), y = out(0);
            SandyTensor w{}, b{};
            const bool hasW = inputs.size() > 1, hasB = inputs.size() > 2;
            if (hasW) w = in(1);
            if (hasB) b = in(2);
            const int32_t kind = k.norm() == kir::NormKind::LayerNorm ? 1 : 0;
            return result(sandy_hip_norm(kind, &x, hasW ? &w : nullptr, hasB ? &b : nullptr, k.epsilon(), &y, stream,
                                         err, sizeof err),
                          err);
        }

        case kir::OpKind::RoPEKernel: {
            const auto& k = static_cast<const kir::RoPEKernelOp&>(op);
            if (auto a = arity(inputs, outputs, 1, 1, "rope"); !a) return a;
            auto x = in(0), y = out(0);
            SandyTensor ids{};
            const bool hasIds = inputs.size() > 1;
            if (hasIds) ids = in(1);
            return result(sandy_hip_rope(&x, hasIds ? &ids : nullptr, k.theta(), k.rotaryDim(), k.splitHalf() ? 1 : 0,
                                         &y, stream, err, sizeof err),
                          err);
        }

        case kir::OpKind::AttentionKernel: {
            const auto& k = static_cast<const kir::AttentionKernelOp&>(op);
            if (auto a = arity(inputs, outputs, 3, 1, "attention"); !a) return a;
            auto q = in(0), y = out(0);
            SandyTensor pos{};
            const bool hasPos = inputs.size() > 3;
            if (hasPos) pos = in(3);
            if (inputs[0].paged || (hasPos && inputs[3].paged))
                return make_error("hip attention q and position_offsets must be dense");
            if (inputs[1].paged != inputs[2].paged) return make_error("hip attention k and v must both be paged or dense");
            if (inputs[1].paged) {
                const int rank = inputs[1].view.desc.shape.rank();
                if (inputs[1].growDim != rank - 2 || inputs[2].growDim != rank - 2)
                    return make_error("hip attention paged k and v must grow along the sequence dimension");
                auto kp = to_paged(inputs[1]), vp = to_paged(inputs[2]);
                return result(sandy_hip_attention_paged_view(&q, &kp, &vp, hasPos ? &pos : nullptr, k.window(),
                                                             k.scale(), &y, stream, err, sizeof err),
                              err);
            }
            auto kd = in(1), vd = in(2);
            return result(sandy_hip_attention(&q, &kd, &vd, hasPos ? &pos : nullptr, k.window(), k.scale(), &y, stream,
                                              err, sizeof err),
                          err);
        }

        case kir::OpKind::MoeGatherKernel: {
            const auto& k = static_cast<const kir::MoeGatherKernelOp&>(op);
            if (auto a = arity(inputs, outputs, 3, 4, "moe_gather"); !a) return a;
            auto x = in(0), ids = in(1), w = in(2);
            auto px = out(0), pw = out(1), tok = out(2), offs = out(3);
            return result(sandy_hip_moe_gather(&x, &ids, &w, k.numExperts(), k.topK(), &px, &pw, &tok, &offs, stream,
                                               err, sizeof err),
                          err);
        }

        case kir::OpKind::MoeMatMulKernel: {
            const auto& k = static_cast<const kir::MoeMatMulKernelOp&>(op);
            if (auto a = arity(inputs, outputs, 3, 1, "moe_matmul"); !a) return a;
            auto x = in(0), offs = in(1), w = in(2), y = out(0);
            return result(sandy_hip_moe_matmul(&x, &offs, &w, k.transposeRhs() ? 1 : 0, &y, stream, err, sizeof err),
                          err);
        }

        case kir::OpKind::MoeScatterSumKernel: {
            // the fourth input is the reference tensor that fixes the output shape
            if (auto a = arity(inputs, outputs, 3, 1, "moe_scatter_sum"); !a) return a;
            auto packed = in(0), w = in(1), tok = in(2), y = out(0);
            return result(sandy_hip_moe_scatter_sum(&packed, &w, &tok, &y, stream, err, sizeof err), err);
        }

        case kir::OpKind::SlidingQueryKeyScoreKernel:
            return make_error("hip device: sliding_query_key_score is not part of this backend");
    }
    return make_error("hip device: unsupported kernel");
}

} // namespace sandy::device
