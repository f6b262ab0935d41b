// ref_shim.cpp -- extern "C" entry points over the reference's own CPU math
// (sandy::core in src/core/TensorCalc.h), so the oracle restatement can be
// checked against the real reference on identical inputs.  TEST
// INFRASTRUCTURE ONLY: built by oracle/Makefile into oracle/_ref/ from the
// reference sources where they lie; never part of the product path.
//
// Signatures mirror sandy_oracle.h (prefix ref_ instead of oracle_).
#include "ShapeUtil.h"
#include "TensorCalc.h"

#include <cstdint>
#include <cstdio>
#include <cstring>
#include <span>
#include <string>
#include <vector>

using sandy::core::DType;
using sandy::core::MutableTensorRef;
using sandy::core::Shape;
using sandy::core::TensorDesc;
using sandy::core::TensorRef;

namespace {

thread_local std::string g_err;

DType dt(int code) { return static_cast<DType>(code); }

TensorRef in(const void* p, std::vector<int64_t> dims, int dtype) {
    TensorDesc desc(Shape(dims), dt(dtype));
    int64_t n = desc.shape.numel();
    auto bytes = std::span<const uint8_t>(
        static_cast<const uint8_t*>(p), static_cast<size_t>(n) * sandy::core::dtype_size(dt(dtype)));
    return sandy::core::make_tensor_ref(desc, bytes).take();
}

MutableTensorRef outref(void* p, std::vector<int64_t> dims, int dtype) {
    TensorDesc desc(Shape(dims), dt(dtype));
    int64_t n = desc.shape.numel();
    auto bytes = std::span<uint8_t>(
        static_cast<uint8_t*>(p), static_cast<size_t>(n) * sandy::core::dtype_size(dt(dtype)));
    return sandy::core::make_mutable_tensor_ref(desc, bytes).take();
}

int ret(const Result<void>& r) {
    if (r) return 0;
    g_err = r.error();
    return -1;
}

} // namespace

extern "C" {

const char* ref_last_error(void) { return g_err.c_str(); }

int ref_rms_norm(const void* x, const void* w, void* out, int dtype, int64_t rows, int64_t cols, float eps) {
    auto xr = in(x, {rows, cols}, dtype);
    auto o = outref(out, {rows, cols}, dtype);
    if (w) return ret(sandy::core::rms_norm(xr, in(w, {cols}, dtype), eps, o));
    return ret(sandy::core::rms_norm(xr, eps, o));
}

int ref_layer_norm(const void* x, const void* w, const void* b, void* out, int dtype,
                   int64_t rows, int64_t cols, float eps) {
    return ret(sandy::core::layer_norm(in(x, {rows, cols}, dtype), in(w, {cols}, dtype),
                                       in(b, {cols}, dtype), eps, outref(out, {rows, cols}, dtype)));
}

int ref_softmax(const void* x, void* out, int dtype, int64_t outer, int64_t axis, int64_t inner) {
    return ret(sandy::core::softmax(in(x, {outer, axis, inner}, dtype), 1,
                                    outref(out, {outer, axis, inner}, dtype)));
}

int ref_sum(const void* x, void* out, int dtype, int64_t outer, int64_t axis, int64_t inner) {
    return ret(sandy::core::sum(in(x, {outer, axis, inner}, dtype), 1, true,
                                outref(out, {outer, 1, inner}, dtype)));
}

int ref_rope(const void* x, const void* pos, int pos_dtype, int64_t pos_count, void* out, int dtype,
             int64_t vectors, int64_t seq, int64_t dim, float theta, int64_t rotary_dim, int split_half) {
    auto xr = in(x, {vectors / seq, seq, dim}, dtype);
    auto o = outref(out, {vectors / seq, seq, dim}, dtype);
    if (pos)
        return ret(sandy::core::rope(xr, in(pos, {pos_count}, pos_dtype), theta, rotary_dim,
                                     split_half != 0, o));
    return ret(sandy::core::rope(xr, theta, rotary_dim, split_half != 0, o));
}

int ref_attention(const void* q, const void* k, const void* v, const void* pos, int pos_dtype,
                  void* out, int dtype, int64_t batch, int64_t heads, int64_t kv_heads, int64_t tq,
                  int64_t tk, int64_t head_dim, int64_t window, float scale) {
    auto qr = in(q, {batch, heads, tq, head_dim}, dtype);
    auto kr = in(k, {batch, kv_heads, tk, head_dim}, dtype);
    auto vr = in(v, {batch, kv_heads, tk, head_dim}, dtype);
    auto o = outref(out, {batch, heads, tq, head_dim}, dtype);
    if (pos)
        return ret(sandy::core::attention(qr, kr, vr, in(pos, {batch}, pos_dtype), window, scale, o));
    return ret(sandy::core::attention(qr, kr, vr, window, scale, o));
}

int ref_topk(const void* x, void* values, void* indices, int idx_dtype, int dtype,
             int64_t outer, int64_t axis, int64_t inner, int64_t k) {
    return ret(sandy::core::topk(in(x, {outer, axis, inner}, dtype), k, 1,
                                 outref(values, {outer, k, inner}, dtype),
                                 outref(indices, {outer, k, inner}, idx_dtype)));
}

int ref_embedding(const void* ids, int ids_dtype, int64_t n_ids, const void* weight, int dtype,
                  int64_t vocab, int64_t hidden, void* out) {
    return ret(sandy::core::embedding(in(ids, {n_ids}, ids_dtype), in(weight, {vocab, hidden}, dtype),
                                      outref(out, {n_ids, hidden}, dtype)));
}

int ref_moe_gather(const void* x, int dtype, const void* ids, int ids_dtype, const void* w, int w_dtype,
                   int64_t batch, int64_t seq, int64_t hidden, int64_t experts, int64_t top_k,
                   void* packed_x, void* packed_w, void* token_ids, int tok_dtype,
                   void* offsets, int off_dtype) {
    int64_t rows = seq * top_k;
    return ret(sandy::core::moe_gather(
        in(x, {batch, seq, hidden}, dtype), in(ids, {batch, seq, top_k}, ids_dtype),
        in(w, {batch, seq, top_k}, w_dtype), experts, top_k,
        outref(packed_x, {batch, rows, hidden}, dtype), outref(packed_w, {batch, rows}, w_dtype),
        outref(token_ids, {batch, rows}, tok_dtype), outref(offsets, {batch, experts + 1}, off_dtype)));
}

int ref_moe_matmul(const void* x, const void* offsets, int off_dtype, const void* weight, int dtype,
                   int64_t batch, int64_t rows, int64_t in_features, int64_t experts,
                   int64_t out_features, int transpose_rhs, void* out) {
    std::vector<int64_t> wdims = transpose_rhs
        ? std::vector<int64_t>{experts, out_features, in_features}
        : std::vector<int64_t>{experts, in_features, out_features};
    return ret(sandy::core::moe_matmul(
        in(x, {batch, rows, in_features}, dtype), in(offsets, {batch, experts + 1}, off_dtype),
        in(weight, wdims, dtype), transpose_rhs != 0, outref(out, {batch, rows, out_features}, dtype)));
}

int ref_moe_scatter_sum(const void* packed, const void* w, const void* token_ids, int tok_dtype,
                        int dtype, int64_t batch, int64_t rows, int64_t hidden, int64_t seq, void* out) {
    return ret(sandy::core::moe_scatter_sum(
        in(packed, {batch, rows, hidden}, dtype), in(w, {batch, rows}, dtype),
        in(token_ids, {batch, rows}, tok_dtype), outref(out, {batch, seq, hidden}, dtype)));
}

int ref_binary(int op, const void* lhs, const int64_t* lshape, int lrank, const void* rhs,
               const int64_t* rshape, int rrank, void* out, const int64_t* oshape, int orank, int dtype) {
    auto l = in(lhs, std::vector<int64_t>(lshape, lshape + lrank), dtype);
    auto r = in(rhs, std::vector<int64_t>(rshape, rshape + rrank), dtype);
    auto o = outref(out, std::vector<int64_t>(oshape, oshape + orank), dtype);
    switch (op) {
        case 0: return ret(sandy::core::add(l, r, o));
        case 1: return ret(sandy::core::mul(l, r, o));
        case 2: return ret(sandy::core::div(l, r, o));
    }
    g_err = "unknown binary op";
    return -1;
}

int ref_unary(int op, const void* x, void* out, int dtype, int64_t n) {
    auto xr = in(x, {n}, dtype);
    auto o = outref(out, {n}, dtype);
    switch (op) {
        case 10: return ret(sandy::core::relu(xr, o));
        case 11: return ret(sandy::core::sqrt(xr, o));
        case 12: return ret(sandy::core::tanh(xr, o));
    }
    g_err = "unknown unary op";
    return -1;
}

int ref_matmul(const void* lhs, const int64_t* ldims, int lrank, const void* rhs, const int64_t* rdims, int rrank,
               int transpose_lhs, int transpose_rhs, void* out, int dtype) {
    std::vector<int64_t> ld(ldims, ldims + lrank), rd(rdims, rdims + rrank);
    std::vector<int64_t> lb(ld.begin(), ld.end() - 2), rb(rd.begin(), rd.end() - 2);
    auto bs = sandy::core::matmul_batch_shape(Shape(lb), Shape(rb));
    if (!bs) {
        g_err = bs.error();
        return -1;
    }
    std::vector<int64_t> od = bs.take().dims();
    od.push_back(ld[lrank - (transpose_lhs ? 1 : 2)]);
    od.push_back(rd[rrank - (transpose_rhs ? 2 : 1)]);
    return ret(sandy::core::matmul(in(lhs, ld, dtype), in(rhs, rd, dtype), transpose_lhs != 0, transpose_rhs != 0,
                                   outref(out, od, dtype)));
}

int ref_linear(const void* x, const void* w, const void* b, void* out, int dtype, int64_t rows,
               int64_t in_features, int64_t out_features) {
    return ret(sandy::core::linear(in(x, {rows, in_features}, dtype), in(w, {out_features, in_features}, dtype),
                                   in(b, {out_features}, dtype), outref(out, {rows, out_features}, dtype)));
}

} // extern "C"
