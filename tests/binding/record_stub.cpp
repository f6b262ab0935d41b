// record_stub.cpp -- a recording stand-in for libsandyrt_hip's C ABI, so the
// reference-side binding (sandyrt_amd/reference_binding/HipKernelDispatch.cpp)
// can be executed on a machine without a GPU.  Every entry point the binding
// calls appends one JSON object to the call log -- its name and every
// descriptor it received (null where the binding passed NULL) -- and returns
// SANDY_OK, except that a stream equal to kFailStream makes the call fail
// with a fixed message (to check that errors come back as the binding's
// Result).  sandy_hip_paged_stage answers with a dense descriptor whose data
// address is kStagedBase + slot.
#include "sandyrt_hip.h"

#include <cstdio>
#include <sstream>
#include <string>
#include <vector>

std::vector<std::string> g_calls;
extern void* const kFailStream;
void* const kFailStream = reinterpret_cast<void*>(0xdead);
const uintptr_t kStagedBase = 0x5000000;

namespace {

std::string hex(const void* p) {
    std::ostringstream os;
    os << '"' << std::hex << reinterpret_cast<uintptr_t>(p) << '"';
    return os.str();
}

template <typename T>
std::string arr(const T* v, int n) {
    std::ostringstream os;
    os << '[';
    for (int i = 0; i < n; i++) os << (i ? "," : "") << v[i];
    os << ']';
    return os.str();
}

std::string t(const SandyTensor* x) {
    if (!x) return "null";
    std::ostringstream os;
    os << "{\"data\":" << hex(x->data) << ",\"dtype\":" << x->dtype << ",\"dims\":" << arr(x->dims, x->rank)
       << ",\"strides\":" << arr(x->strides, x->rank) << ",\"offset\":" << x->storage_offset << '}';
    return os.str();
}

std::string pv(const SandyPagedView* x) {
    if (!x) return "null";
    std::ostringstream os;
    os << "{\"pages\":" << hex(x->pages) << ",\"dtype\":" << x->dtype << ",\"dims\":" << arr(x->dims, x->rank)
       << ",\"page_size\":" << x->page_size << ",\"page_count\":" << x->page_count << '}';
    return os.str();
}

std::string pt(const SandyPagedTensor* x) {
    if (!x) return "null";
    std::ostringstream os;
    os << "{\"pages\":" << hex(x->pages) << ",\"dtype\":" << x->dtype << ",\"dims\":" << arr(x->dims, x->rank)
       << ",\"grow_dim\":" << x->grow_dim << ",\"page_size\":" << x->page_size << ",\"page_count\":" << x->page_count
       << '}';
    return os.str();
}

int rec(const char* name, const std::string& fields, void* stream, char* err, size_t cap) {
    g_calls.push_back(std::string("{\"call\":\"") + name + "\"" + fields + "}");
    if (stream == kFailStream) {
        std::snprintf(err, cap, "%s failed in the stub", name);
        return SANDY_ERR_INVALID;
    }
    if (err && cap) err[0] = 0;
    return SANDY_OK;
}

std::string f(const char* k, const std::string& v) { return std::string(",\"") + k + "\":" + v; }
std::string f(const char* k, double v) {
    std::ostringstream os;
    os.precision(17);
    os << ",\"" << k << "\":" << v;
    return os.str();
}
std::string f(const char* k, int64_t v) { return std::string(",\"") + k + "\":" + std::to_string(v); }

} // namespace

extern "C" {

int sandy_hip_paged_stage(const SandyPagedTensor* src, int32_t slot, SandyTensor* dense, void* stream, char* err,
                          size_t cap) {
    *dense = SandyTensor{};
    dense->data = reinterpret_cast<void*>(kStagedBase + static_cast<uintptr_t>(slot));
    dense->dtype = src->dtype;
    dense->rank = src->rank;
    int64_t s = 1;
    for (int i = src->rank - 1; i >= 0; i--) {
        dense->dims[i] = src->dims[i];
        dense->strides[i] = s;
        s *= src->dims[i];
    }
    return rec("sandy_hip_paged_stage", f("src", pt(src)) + f("slot", int64_t{slot}), stream, err, cap);
}

int sandy_hip_layout_transform(const SandyTensor* in, const SandyTensor* out, int32_t kind, void* stream, char* err,
                               size_t cap) {
    return rec("sandy_hip_layout_transform", f("in", t(in)) + f("out", t(out)) + f("kind", int64_t{kind}), stream, err,
               cap);
}

int sandy_hip_elementwise(const SandyScalarNode* nodes, int32_t node_count, uint32_t result, const SandyTensor* inputs,
                          const int32_t* broadcast, int32_t input_count, const SandyTensor* out, void* stream,
                          char* err, size_t cap) {
    std::ostringstream ns;
    ns << '[';
    for (int i = 0; i < node_count; i++) {
        const auto& n = nodes[i];
        ns << (i ? "," : "") << "{\"id\":" << n.id << ",\"op\":" << n.op << ",\"dtype\":" << n.dtype
           << ",\"input\":" << n.input_index << ",\"constant\":" << n.constant << ",\"operands\":"
           << arr(n.operands, n.operand_count) << '}';
    }
    ns << ']';
    std::ostringstream is;
    is << '[';
    for (int i = 0; i < input_count; i++) is << (i ? "," : "") << t(&inputs[i]);
    is << ']';
    return rec("sandy_hip_elementwise",
               f("nodes", ns.str()) + f("result", int64_t{result}) + f("inputs", is.str()) +
                   f("broadcast", arr(broadcast, input_count)) + f("out", t(out)),
               stream, err, cap);
}

int sandy_hip_reduce_sum(const SandyTensor* x, int64_t axis, int32_t keep_dims, const SandyTensor* out, void* stream,
                         char* err, size_t cap) {
    return rec("sandy_hip_reduce_sum", f("x", t(x)) + f("axis", axis) + f("keep_dims", int64_t{keep_dims}) + f("out", t(out)),
               stream, err, cap);
}

int sandy_hip_linear(const SandyTensor* x, const SandyTensor* w, const SandyTensor* b, const SandyTensor* out,
                     void* stream, char* err, size_t cap) {
    return rec("sandy_hip_linear", f("x", t(x)) + f("weight", t(w)) + f("bias", t(b)) + f("out", t(out)), stream, err,
               cap);
}

int sandy_hip_matmul(const SandyTensor* l, const SandyTensor* r, int32_t tl, int32_t tr, const SandyTensor* out,
                     void* stream, char* err, size_t cap) {
    return rec("sandy_hip_matmul",
               f("lhs", t(l)) + f("rhs", t(r)) + f("transpose_lhs", int64_t{tl}) + f("transpose_rhs", int64_t{tr}) +
                   f("out", t(out)),
               stream, err, cap);
}

int sandy_hip_gather(const SandyTensor* ids, const SandyTensor* table, const SandyTensor* out, void* stream, char* err,
                     size_t cap) {
    return rec("sandy_hip_gather", f("ids", t(ids)) + f("table", t(table)) + f("out", t(out)), stream, err, cap);
}

int sandy_hip_softmax(const SandyTensor* x, int64_t axis, const SandyTensor* out, void* stream, char* err, size_t cap) {
    return rec("sandy_hip_softmax", f("x", t(x)) + f("axis", axis) + f("out", t(out)), stream, err, cap);
}

int sandy_hip_topk(const SandyTensor* x, int64_t k, int64_t axis, const SandyTensor* values, const SandyTensor* indices,
                   void* stream, char* err, size_t cap) {
    return rec("sandy_hip_topk",
               f("x", t(x)) + f("k", k) + f("axis", axis) + f("values", t(values)) + f("indices", t(indices)), stream,
               err, cap);
}

int sandy_hip_norm(int32_t kind, const SandyTensor* x, const SandyTensor* w, const SandyTensor* b, double eps,
                   const SandyTensor* out, void* stream, char* err, size_t cap) {
    return rec("sandy_hip_norm",
               f("kind", int64_t{kind}) + f("x", t(x)) + f("weight", t(w)) + f("bias", t(b)) + f("epsilon", eps) +
                   f("out", t(out)),
               stream, err, cap);
}

int sandy_hip_rope(const SandyTensor* x, const SandyTensor* ids, double theta, int64_t rotary_dim, int32_t split_half,
                   const SandyTensor* out, void* stream, char* err, size_t cap) {
    return rec("sandy_hip_rope",
               f("x", t(x)) + f("position_ids", t(ids)) + f("theta", theta) + f("rotary_dim", rotary_dim) +
                   f("split_half", int64_t{split_half}) + f("out", t(out)),
               stream, err, cap);
}

int sandy_hip_attention(const SandyTensor* q, const SandyTensor* k, const SandyTensor* v, const SandyTensor* pos,
                        int64_t window, double scale, const SandyTensor* out, void* stream, char* err, size_t cap) {
    return rec("sandy_hip_attention",
               f("q", t(q)) + f("k", t(k)) + f("v", t(v)) + f("position_offsets", t(pos)) + f("window", window) +
                   f("scale", scale) + f("out", t(out)),
               stream, err, cap);
}

int sandy_hip_attention_paged_view(const SandyTensor* q, const SandyPagedView* k, const SandyPagedView* v,
                                   const SandyTensor* pos, int64_t window, double scale, const SandyTensor* out,
                                   void* stream, char* err, size_t cap) {
    return rec("sandy_hip_attention_paged_view",
               f("q", t(q)) + f("k", pv(k)) + f("v", pv(v)) + f("position_offsets", t(pos)) + f("window", window) +
                   f("scale", scale) + f("out", t(out)),
               stream, err, cap);
}

int sandy_hip_moe_gather(const SandyTensor* x, const SandyTensor* ids, const SandyTensor* w, int64_t experts,
                         int64_t top_k, const SandyTensor* px, const SandyTensor* pw, const SandyTensor* tok,
                         const SandyTensor* offs, void* stream, char* err, size_t cap) {
    return rec("sandy_hip_moe_gather",
               f("x", t(x)) + f("topk_ids", t(ids)) + f("topk_weights", t(w)) + f("num_experts", experts) +
                   f("top_k", top_k) + f("packed_x", t(px)) + f("packed_weights", t(pw)) + f("token_ids", t(tok)) +
                   f("expert_offsets", t(offs)),
               stream, err, cap);
}

int sandy_hip_moe_matmul(const SandyTensor* x, const SandyTensor* offs, const SandyTensor* w, int32_t tr,
                         const SandyTensor* out, void* stream, char* err, size_t cap) {
    return rec("sandy_hip_moe_matmul",
               f("x", t(x)) + f("expert_offsets", t(offs)) + f("weight", t(w)) + f("transpose_rhs", int64_t{tr}) +
                   f("out", t(out)),
               stream, err, cap);
}

int sandy_hip_moe_scatter_sum(const SandyTensor* packed, const SandyTensor* w, const SandyTensor* tok,
                              const SandyTensor* out, void* stream, char* err, size_t cap) {
    return rec("sandy_hip_moe_scatter_sum",
               f("packed_out", t(packed)) + f("packed_weights", t(w)) + f("token_ids", t(tok)) + f("out", t(out)),
               stream, err, cap);
}

}  // extern "C"
