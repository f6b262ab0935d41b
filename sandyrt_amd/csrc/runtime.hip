// runtime.hip -- per-device state of the backend: the sticky device error
// word and grow-only workspaces.  The reference allocates temporaries with
// cudaMallocAsync on every launch (CudaAttentionKernels.cu:496-503,
// CudaTopKKernels.cu:558-567) and reads error flags back with a host sync per
// launch (CudaRoPEKernels.cu:310-333); here both live for the process and the
// flags are read only when the caller asks (sandy_hip_take_device_errors).
#include "common.h"

#include <mutex>

namespace sandy_hip {

namespace {

constexpr int kMaxDevices = 64;
constexpr int kSlots = kPagedStageSlot0 + SANDY_HIP_PAGED_STAGE_SLOTS;

struct DeviceState {
    uint32_t* error_word = nullptr;
    void* ws[kSlots] = {};
    size_t ws_bytes[kSlots] = {};
    void* ctr[kSlots] = {};
    size_t ctr_bytes[kSlots] = {};
};

std::mutex g_mu;
DeviceState g_dev[kMaxDevices];

// The sticky error word of each device lives in this file-scope device array
// (zero when the module loads; word 0 is used), so that no entry point has to
// allocate for it.  Each GPU holds its own copy; host code uses the address
// hipGetSymbolAddress returns for the current device, never the name.
static __device__ __align__(256) uint32_t error_words[64];

int current_device(Err e, int* dev) {
    hipError_t st = hipGetDevice(dev);
    if (st != hipSuccess) return fail(e, SANDY_ERR_HIP, "hipGetDevice: %s", hipGetErrorString(st));
    if (*dev < 0 || *dev >= kMaxDevices) return fail(e, SANDY_ERR_HIP, "device ordinal %d out of range", *dev);
    return SANDY_OK;
}

} // namespace

uint32_t* device_error_word(Err e, int* status) {
    int dev = 0;
    *status = current_device(e, &dev);
    if (*status) return nullptr;
    std::lock_guard<std::mutex> lock(g_mu);
    DeviceState& s = g_dev[dev];
    if (!s.error_word) {
        void* p = nullptr;
        hipError_t st = hipGetSymbolAddress(&p, HIP_SYMBOL(error_words));
        if (st != hipSuccess) {
            *status = fail(e, SANDY_ERR_HIP, "device error word: %s", hipGetErrorString(st));
            return nullptr;
        }
        s.error_word = static_cast<uint32_t*>(p);
    }
    return s.error_word;
}

void* device_workspace(int slot, size_t bytes, hipStream_t stream, Err e, int* status) {
    int dev = 0;
    *status = current_device(e, &dev);
    if (*status) return nullptr;
    if (bytes == 0) bytes = 256;
    std::lock_guard<std::mutex> lock(g_mu);
    DeviceState& s = g_dev[dev];
    if (s.ws_bytes[slot] < bytes) {
        if (s.ws[slot]) {
            // earlier work on any stream may still read the old buffer
            hipDeviceSynchronize();
            hipFree(s.ws[slot]);
            s.ws[slot] = nullptr;
            s.ws_bytes[slot] = 0;
        }
        size_t grown = bytes + bytes / 4;
        hipError_t st = hipMalloc(&s.ws[slot], grown);
        if (st != hipSuccess) {
            *status = fail(e, SANDY_ERR_HIP, "workspace allocation of %zu bytes: %s", grown, hipGetErrorString(st));
            return nullptr;
        }
        s.ws_bytes[slot] = grown;
    }
    (void)stream;
    return s.ws[slot];
}

void* device_counters(int slot, size_t bytes, hipStream_t stream, Err e, int* status) {
    int dev = 0;
    *status = current_device(e, &dev);
    if (*status) return nullptr;
    if (bytes == 0) bytes = 256;
    std::lock_guard<std::mutex> lock(g_mu);
    DeviceState& s = g_dev[dev];
    if (s.ctr_bytes[slot] < bytes) {
        if (s.ctr[slot]) {
            hipDeviceSynchronize();
            hipFree(s.ctr[slot]);
            s.ctr[slot] = nullptr;
            s.ctr_bytes[slot] = 0;
        }
        size_t grown = bytes + bytes / 4;
        hipError_t st = hipMalloc(&s.ctr[slot], grown);
        if (st == hipSuccess) st = hipMemset(s.ctr[slot], 0, grown);
        if (st == hipSuccess) st = hipDeviceSynchronize();
        if (st != hipSuccess) {
            *status = fail(e, SANDY_ERR_HIP, "counter allocation of %zu bytes: %s", grown, hipGetErrorString(st));
            return nullptr;
        }
        s.ctr_bytes[slot] = grown;
    }
    (void)stream;
    return s.ctr[slot];
}

} // namespace sandy_hip

using namespace sandy_hip;

extern "C" const char* sandy_hip_version(void) { return "sandyrt-hip 0.1.0 gfx950"; }

extern "C" int sandy_hip_take_device_errors(void* stream, uint32_t* flags, char* err, size_t err_cap) {
    Err e{err, err_cap};
    int status = 0;
    uint32_t* word = device_error_word(e, &status);
    if (status) return status;
    hipStream_t s = static_cast<hipStream_t>(stream);
    uint32_t host = 0;
    SANDY_HIP_TRY(hipStreamSynchronize(s), e, "hipStreamSynchronize");
    SANDY_HIP_TRY(hipMemcpy(&host, word, sizeof(host), hipMemcpyDeviceToHost), e, "read device error word");
    SANDY_HIP_TRY(hipMemset(word, 0, sizeof(uint32_t)), e, "clear device error word");
    if (flags) *flags = host;
    if (host & SANDY_DEVERR_EXPERT_ID) return fail(e, SANDY_ERR_INVALID, "moe_gather topk expert id out of range");
    if (host & SANDY_DEVERR_TOKEN_ID) return fail(e, SANDY_ERR_INVALID, "moe_scatter_sum token id out of range");
    if (host & SANDY_DEVERR_POSITION) return fail(e, SANDY_ERR_INVALID, "rope position_ids must be non-negative");
    if (host & SANDY_DEVERR_GATHER_ID) return fail(e, SANDY_ERR_INVALID, "embedding id out of range");
    if (host & SANDY_DEVERR_OFFSETS) return fail(e, SANDY_ERR_INVALID, "moe_matmul invalid expert offsets");
    if (host & SANDY_DEVERR_BLOCK) return fail(e, SANDY_ERR_INVALID, "paged attention block id outside the pool");
    if (host & SANDY_DEVERR_ATTN_POS) return fail(e, SANDY_ERR_INVALID, "attention position_offsets must be non-negative");
    return ok(e);
}
