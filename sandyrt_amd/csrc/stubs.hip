// stubs.hip -- entry points whose kernels are not written yet report
// SANDY_ERR_UNSUPPORTED.
#include "common.h"
using namespace sandy_hip;
#define STUB(name, ...) extern "C" int name(__VA_ARGS__, void*, char* err, size_t cap) { return fail(Err{err, cap}, SANDY_ERR_UNSUPPORTED, #name " is not implemented"); }
