// stubs.hip -- entry points whose kernels are not written yet report
// SANDY_ERR_UNSUPPORTED.
#include "common.h"
using namespace sandy_hip;
#define STUB(name, ...) extern "C" int name(__VA_ARGS__, void*, char* err, size_t cap) { return fail(Err{err, cap}, SANDY_ERR_UNSUPPORTED, #name " is not implemented"); }
STUB(sandy_hip_topk, const SandyTensor*, int64_t, int64_t, const SandyTensor*, const SandyTensor*)
STUB(sandy_hip_moe_gather, const SandyTensor*, const SandyTensor*, const SandyTensor*, int64_t, int64_t, const SandyTensor*, const SandyTensor*, const SandyTensor*, const SandyTensor*)
STUB(sandy_hip_moe_matmul, const SandyTensor*, const SandyTensor*, const SandyTensor*, int32_t, const SandyTensor*)
STUB(sandy_hip_moe_scatter_sum, const SandyTensor*, const SandyTensor*, const SandyTensor*, const SandyTensor*)
