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
// headers (KernelIR.h, DeviceTypes.h, Result.h, Tensor.h) and sandyrt_hip.h.
// tests/test_binding.py builds it with the reference's src/ir and src/core
// sources and a recording stand-in of the C ABI, and runs one op of every
// OpKind through it.
#include "HipKernelDispatch.h"

#include <cstdint>
#include <span>
#include <string>
#include <vector>

namespace sandy::device {

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

// The C ABI's status as the reference's Result: the message is already worded
// like the reference's errors.
Result<void> result(int rc, const char* err) {
    if (rc == SANDY_OK) return {};
    return make_error(std::string(err));
}

// A paged view is described by its logical shape; the reference rejects any
// other view of one (pack_tensor_arg, CudaKernelUtils.cuh:303-306).
Result<void> paged_view_ok(const HipDeviceBufferView& b) {
    const auto& v = b.view;
    int64_t expected = 1;
    const int rank = v.desc.shape.rank();
    if (rank > SANDY_HIP_MAX_RANK) return make_error("hip tensor rank exceeds kernel max rank");
    if (static_cast<int>(v.strides.size()) != rank) return make_error("hip tensor strides rank mismatch");
    for (int d = rank - 1; d >= 0; --d) {
        if (v.desc.shape.dim(d) != 1 && v.strides[static_cast<size_t>(d)] != expected)
            return make_error("hip paged tensor view must be contiguous");
        expected *= v.desc.shape.dim(d);
    }
    if (v.storageOffset != 0) return make_error("hip paged tensor storage offset must be zero");
    return {};
}

SandyPagedTensor to_paged_tensor(const HipDeviceBufferView& b) {
    SandyPagedTensor p{};
    p.pages = b.data;
    p.dtype = static_cast<int32_t>(b.view.desc.dtype);
    p.rank = b.view.desc.shape.rank();
    for (int i = 0; i < p.rank && i < SANDY_HIP_MAX_RANK; ++i) p.dims[i] = b.view.desc.shape.dim(i);
    p.grow_dim = b.growDim;
    p.page_size = b.pageSize;
    p.page_count = b.pageCount;
    return p;
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

// The inputs of a family that reads paged operands (the reference's
// load_float / load_int, CudaKernelUtils.cuh:82-157): a dense input is passed
// as it is, a paged one is gathered into the library's staging slot of its
// input index first (sandy_hip_paged_stage), on the launch stream.
struct StagedInputs {
    std::span<const HipDeviceBufferView> views;
    void* stream;
    std::vector<SandyTensor> dense;

    Result<void> stage() {
        dense.resize(views.size());
        for (size_t i = 0; i < views.size(); ++i) {
            if (!views[i].paged) {
                dense[i] = to_tensor(views[i]);
                continue;
            }
            if (i >= SANDY_HIP_PAGED_STAGE_SLOTS) return make_error("hip kernel has too many paged inputs");
            if (auto v = paged_view_ok(views[i]); !v) return v;
            auto p = to_paged_tensor(views[i]);
            char err[512] = {0};
            if (auto r = result(sandy_hip_paged_stage(&p, static_cast<int32_t>(i), &dense[i], stream, err, sizeof err),
                                err);
                !r)
                return r;
        }
        return {};
    }
};

Result<void> no_paged(std::span<const HipDeviceBufferView> views, const std::string& message) {
    for (const auto& v : views)
        if (v.paged) return make_error(message);
    return {};
}

// The MoE families name the operand that is paged (CudaGatherKernels.cu:127-132,
// CudaMoeScatterSumKernels.cu:26-31).
Result<void> no_paged_named(std::span<const HipDeviceBufferView> views, std::span<const char* const> names,
                            const char* kernel) {
    for (size_t i = 0; i < views.size() && i < names.size(); ++i)
        if (views[i].paged) return make_error(std::string("hip ") + kernel + " " + names[i] + " cannot be paged");
    return {};
}

Result<void> arity(std::span<const HipDeviceBufferView> in, std::span<const HipDeviceBufferView> out, size_t minIn,
                   size_t minOut, const char* kernel) {
    if (in.size() < minIn) return make_error(std::string("hip ") + kernel + " input arity mismatch");
    if (out.size() < minOut) return make_error(std::string("hip ") + kernel + " output arity mismatch");
    return {};
}

} // namespace

Result<void> hip_run_kernel(const kir::Op& op, std::span<const HipDeviceBufferView> inputs,
                            std::span<const HipDeviceBufferView> outputs, void* stream) {
    char err[512] = {0};
    // outputs are dense tensor views (CudaDevice.cpp:497-503)
    for (const auto& o : outputs)
        if (o.paged) return make_error("hip device kernel output must be a dense tensor view");
    auto out = [&](size_t i) { return to_tensor(outputs[i]); };
    StagedInputs staged{inputs, stream, {}};
    auto in = [&](size_t i) { return staged.dense[i]; };

    switch (op.kind()) {
        case kir::OpKind::Input:
        case kir::OpKind::TensorTupleCreate:
        case kir::OpKind::DeviceTransfer:
        case kir::OpKind::PagedAppend:
            return make_error("hip device cannot run boundary op");

        case kir::OpKind::LayoutTransform: {
            const auto& k = static_cast<const kir::LayoutTransformOp&>(op);
            if (auto a = arity(inputs, outputs, 1, 1, "layout_transform"); !a) return a;
            if (auto d = no_paged(inputs, "hip layout_transform does not support paged tensors"); !d) return d;
            auto x = to_tensor(inputs[0]), y = out(0);
            return result(sandy_hip_layout_transform(&x, &y, static_cast<int32_t>(k.transform()), stream, err,
                                                     sizeof err),
                          err);
        }

        case kir::OpKind::ElementwiseKernel: {
            const auto& k = static_cast<const kir::ElementwiseKernelOp&>(op);
            if (auto a = arity(inputs, outputs, k.elementwiseInputs().size(), 1, "elementwise"); !a) return a;
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
            if (auto r = staged.stage(); !r) return r;
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
            if (auto r = staged.stage(); !r) return r;
            auto x = in(0), y = out(0);
            return result(sandy_hip_reduce_sum(&x, k.axes()[0], k.keepDims() ? 1 : 0, &y, stream, err, sizeof err),
                          err);
        }

        case kir::OpKind::LinearKernel: {
            if (auto a = arity(inputs, outputs, 2, 1, "linear"); !a) return a;
            if (auto d = no_paged(inputs, "hip linear does not support paged tensor operands"); !d) return d;
            auto x = to_tensor(inputs[0]), w = to_tensor(inputs[1]), y = out(0);
            SandyTensor b{};
            const bool hasBias = inputs.size() > 2;
            if (hasBias) b = to_tensor(inputs[2]);
            return result(sandy_hip_linear(&x, &w, hasBias ? &b : nullptr, &y, stream, err, sizeof err), err);
        }

        case kir::OpKind::MatMulKernel: {
            const auto& k = static_cast<const kir::MatMulKernelOp&>(op);
            if (auto a = arity(inputs, outputs, 2, 1, "matmul"); !a) return a;
            if (auto d = no_paged(inputs, "hip matmul does not support paged tensor operands"); !d) return d;
            auto lhs = to_tensor(inputs[0]), rhs = to_tensor(inputs[1]), y = out(0);
            return result(sandy_hip_matmul(&lhs, &rhs, k.transposeLhs() ? 1 : 0, k.transposeRhs() ? 1 : 0, &y, stream,
                                           err, sizeof err),
                          err);
        }

        case kir::OpKind::GatherKernel: {
            if (auto a = arity(inputs, outputs, 2, 1, "gather"); !a) return a;
            if (auto r = staged.stage(); !r) return r;
            auto ids = in(0), table = in(1), y = out(0);
            return result(sandy_hip_gather(&ids, &table, &y, stream, err, sizeof err), err);
        }

        case kir::OpKind::SoftmaxKernel: {
            const auto& k = static_cast<const kir::SoftmaxKernelOp&>(op);
            if (auto a = arity(inputs, outputs, 1, 1, "softmax"); !a) return a;
            if (auto r = staged.stage(); !r) return r;
            auto x = in(0), y = out(0);
            return result(sandy_hip_softmax(&x, k.axis(), &y, stream, err, sizeof err), err);
        }

        case kir::OpKind::TopKKernel: {
            const auto& k = static_cast<const kir::TopKKernelOp&>(op);
            if (auto a = arity(inputs, outputs, 1, 2, "topk"); !a) return a;
            if (auto d = no_paged(inputs, "hip topk does not support paged tensor operands"); !d) return d;
            auto x = to_tensor(inputs[0]), values = out(0), indices = out(1);
            return result(sandy_hip_topk(&x, k.k(), k.axis(), &values, &indices, stream, err, sizeof err), err);
        }

        case kir::OpKind::NormKernel: {
            const auto& k = static_cast<const kir::NormKernelOp&>(op);
            if (auto a = arity(inputs, outputs, 1, 1, "norm"); !a) return a;
            if (auto r = staged.stage(); !r) return r;
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
            if (auto r = staged.stage(); !r) return r;
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
            const bool hasPos = inputs.size() > 3;
            const int rank = inputs[1].view.desc.shape.rank();
            // K and V paged along the key dimension of a rank-3/4 view: the paged
            // decode kernels read the pages themselves
            const bool pagedKv = inputs[1].paged && inputs[2].paged && (rank == 3 || rank == 4) &&
                                 inputs[2].view.desc.shape.rank() == rank && inputs[1].growDim == rank - 2 &&
                                 inputs[2].growDim == rank - 2;
            if (pagedKv) {
                if (auto v = paged_view_ok(inputs[1]); !v) return v;
                if (auto v = paged_view_ok(inputs[2]); !v) return v;
                // q and positions may still be paged: staged like any other input
                HipDeviceBufferView rest[2] = {inputs[0], hasPos ? inputs[3] : HipDeviceBufferView{}};
                StagedInputs qs{std::span<const HipDeviceBufferView>(rest, hasPos ? 2 : 1), stream, {}};
                if (auto r = qs.stage(); !r) return r;
                auto q = qs.dense[0], y = out(0);
                SandyTensor pos = hasPos ? qs.dense[1] : SandyTensor{};
                auto kp = to_paged(inputs[1]), vp = to_paged(inputs[2]);
                return result(sandy_hip_attention_paged_view(&q, &kp, &vp, hasPos ? &pos : nullptr, k.window(),
                                                             k.scale(), &y, stream, err, sizeof err),
                              err);
            }
            if (auto r = staged.stage(); !r) return r;
            auto q = in(0), kd = in(1), vd = in(2), y = out(0);
            SandyTensor pos = hasPos ? in(3) : SandyTensor{};
            return result(sandy_hip_attention(&q, &kd, &vd, hasPos ? &pos : nullptr, k.window(), k.scale(), &y, stream,
                                              err, sizeof err),
                          err);
        }

        case kir::OpKind::MoeGatherKernel: {
            const auto& k = static_cast<const kir::MoeGatherKernelOp&>(op);
            if (auto a = arity(inputs, outputs, 3, 4, "moe_gather"); !a) return a;
            static const char* const inNames[] = {"x", "topk_ids", "topk_weights"};
            if (auto d = no_paged_named(inputs, inNames, "moe_gather"); !d) return d;
            auto x = to_tensor(inputs[0]), ids = to_tensor(inputs[1]), w = to_tensor(inputs[2]);
            auto px = out(0), pw = out(1), tok = out(2), offs = out(3);
            return result(sandy_hip_moe_gather(&x, &ids, &w, k.numExperts(), k.topK(), &px, &pw, &tok, &offs, stream,
                                               err, sizeof err),
                          err);
        }

        case kir::OpKind::MoeMatMulKernel: {
            const auto& k = static_cast<const kir::MoeMatMulKernelOp&>(op);
            if (auto a = arity(inputs, outputs, 3, 1, "moe_matmul"); !a) return a;
            if (auto d = no_paged(inputs, "hip moe_matmul does not support paged tensor operands"); !d) return d;
            auto x = to_tensor(inputs[0]), offs = to_tensor(inputs[1]), w = to_tensor(inputs[2]), y = out(0);
            return result(sandy_hip_moe_matmul(&x, &offs, &w, k.transposeRhs() ? 1 : 0, &y, stream, err, sizeof err),
                          err);
        }

        case kir::OpKind::MoeScatterSumKernel: {
            // the fourth input is the reference tensor that fixes the output shape
            if (auto a = arity(inputs, outputs, 3, 1, "moe_scatter_sum"); !a) return a;
            static const char* const inNames[] = {"packed_out", "packed_weights", "token_ids", "reference"};
            if (auto d = no_paged_named(inputs, inNames, "moe_scatter_sum"); !d) return d;
            auto packed = to_tensor(inputs[0]), w = to_tensor(inputs[1]), tok = to_tensor(inputs[2]), y = out(0);
            return result(sandy_hip_moe_scatter_sum(&packed, &w, &tok, &y, stream, err, sizeof err), err);
        }

        case kir::OpKind::SlidingQueryKeyScoreKernel:
            return make_error("hip device: sliding_query_key_score is not part of this backend");
    }
    return make_error("hip device: unsupported kernel");
}

} // namespace sandy::device
