// hip_device.hip -- the device object: buffers, paged tensor pools with
// device-resident block tables and lengths, one stream, HIP graph capture.
//
// Mirrors the responsibilities of sandy::device::Device
// (src/device/Device.h:27-66) and the CUDA backend's paged storage
// (src/device/cuda/CudaPagedTensor.{h,cpp}).  Differences by design:
//   - a pool is one allocation of pages, pages are int32 block ids (the
//     reference allocates every page separately and keeps a void* page table
//     per tensor, synchronised to the device incrementally);
//   - each pool keeps an int32 block table [max_tensors, max_blocks] and int32
//     grow lengths [max_tensors] on the device; a tensor is a row (slot);
//   - an append is one kernel launch instead of one cudaMemcpyAsync per
//     (prefix, grow) row (CudaPagedTensor.cpp:649-740); the step append reads
//     and advances the lengths on the device, so a decode step needs no host
//     bookkeeping and can be captured in a graph.
// Error wording follows the reference (CpuDevice.cpp:444-554,
// CudaPagedTensor.cpp:30-55,232-258, Device.cpp:13-19).
#include "common.h"
#include "gemm.h"

#include <algorithm>
#include <cmath>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

namespace sandy_hip {
namespace {

constexpr int kMaxStepTensors = 512;

struct PagedPool {
    SandyPagedPoolDesc desc{};
    int64_t prefix = 1, inner = 1;   // elements before / after the grow dim
    int64_t page_elems = 0;          // prefix * page_size * inner
    size_t elem = 0;
    char* pages = nullptr;           // [capacity, prefix, page_size, inner]
    int64_t capacity = 0;
    int64_t used = 0;                // pages ever handed out (high-water mark)
    std::vector<int32_t> free_pages;
    int32_t* table = nullptr;        // device [max_tensors, max_blocks]
    int32_t* host_table = nullptr;   // pinned mirror: source of the table updates
    int32_t* lengths = nullptr;      // device [max_tensors]
    std::vector<int32_t> free_slots;
};

struct PagedTensor {
    uint32_t pool = 0;
    int32_t slot = 0;
    int64_t grow_length = 0;
    std::vector<int32_t> pages;
};

struct StepArgs {
    int32_t slots[kMaxStepTensors];
};

// chunk rows -> pages: one wave per (prefix, grow) row of the chunk
__global__ __launch_bounds__(256) void paged_append_kernel(const char* __restrict__ src, char* __restrict__ pages,
                                                           const int32_t* __restrict__ table_row,
                                                           int32_t* __restrict__ length_slot, int64_t old_len,
                                                           int64_t chunk_len, int64_t prefix, int64_t page_size,
                                                           int64_t row_bytes, int64_t page_bytes) {
    const int lane = threadIdx.x & 63;
    const int64_t r = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    if (r == 0 && threadIdx.x == 0) *length_slot = static_cast<int32_t>(old_len + chunk_len);
    if (r >= prefix * chunk_len) return;
    const int64_t p = r / chunk_len, g = r % chunk_len;
    const int64_t dst_grow = old_len + g;
    const int32_t blk = table_row[dst_grow / page_size];
    const char* s = src + r * row_bytes;
    char* d = pages + blk * page_bytes + (p * page_size + dst_grow % page_size) * row_bytes;
    if ((row_bytes & 15) == 0 && ((reinterpret_cast<uintptr_t>(s) | reinterpret_cast<uintptr_t>(d)) & 15) == 0) {
        for (int64_t o = lane * 16; o < row_bytes; o += 64 * 16)
            *reinterpret_cast<uint4*>(d + o) = *reinterpret_cast<const uint4*>(s + o);
    } else {
        for (int64_t o = lane; o < row_bytes; o += 64) d[o] = s[o];
    }
}

// One grow row of tensor i of a step append (workgroup per row): rows of up
// to 1 KiB, 16-byte multiples at 16-byte aligned addresses (`aligned16`
// covers the rows view and the page pool), are requested before the slot ->
// length -> block-table chain they do not depend on.
__device__ __forceinline__ void append_step_row(const char* __restrict__ rows, char* __restrict__ pages,
                                                const int32_t* __restrict__ table, int32_t* __restrict__ lengths,
                                                int64_t max_blocks, int64_t prefix, int64_t page_size,
                                                int64_t row_bytes, int64_t page_bytes, uint32_t* errw, int i,
                                                int32_t slot, int32_t aligned16) {
    const int lane = threadIdx.x & 63;
    // up to 16 rows of a tensor: this thread's pieces (rows wave + 4j, piece lane)
    const bool vec = aligned16 && (row_bytes & 15) == 0;
    const bool pre = vec && row_bytes <= 1024 && prefix <= 16;
    // (four named registers: an array here was placed in LDS, whose writes
    // waited for the loads)
    uint4 p0{}, p1{}, p2{}, p3{};
    const int w4 = threadIdx.x >> 6;
    if (pre) {
        const int64_t np = row_bytes / 16;
        const int64_t lc = lane < np ? lane : np - 1;
        const char* rb = rows + static_cast<int64_t>(i) * prefix * row_bytes + lc * 16;
        auto at = [&](int64_t p) { return reinterpret_cast<const uint4*>(rb + (p < prefix ? p : prefix - 1) * row_bytes); };
        p0 = *at(w4);
        p1 = *at(w4 + 4);
        p2 = *at(w4 + 8);
        p3 = *at(w4 + 12);
    }
    const int32_t len = lengths[slot];
    __syncthreads();  // every wave has read the length before it advances
    const int32_t page = len / page_size;
    const int32_t blk = page < max_blocks ? table[slot * max_blocks + page] : -1;
    if (blk >= 0 && pre) {
        char* db = pages + blk * page_bytes + (len % page_size) * row_bytes + lane * 16;
        const int64_t pstride = page_size * row_bytes;
        if (lane * 16 < row_bytes) {
            if (w4 < prefix) *reinterpret_cast<uint4*>(db + w4 * pstride) = p0;
            if (w4 + 4 < prefix) *reinterpret_cast<uint4*>(db + (w4 + 4) * pstride) = p1;
            if (w4 + 8 < prefix) *reinterpret_cast<uint4*>(db + (w4 + 8) * pstride) = p2;
            if (w4 + 12 < prefix) *reinterpret_cast<uint4*>(db + (w4 + 12) * pstride) = p3;
        }
    } else if (blk >= 0) {
        for (int64_t p = threadIdx.x >> 6; p < prefix; p += 4) {
            const char* s = rows + (static_cast<int64_t>(i) * prefix + p) * row_bytes;
            char* d = pages + blk * page_bytes + (p * page_size + len % page_size) * row_bytes;
            if (vec) {
                for (int64_t o = lane * 16; o < row_bytes; o += 64 * 16)
                    *reinterpret_cast<uint4*>(d + o) = *reinterpret_cast<const uint4*>(s + o);
            } else {
                for (int64_t o = lane; o < row_bytes; o += 64) d[o] = s[o];
            }
        }
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        if (blk >= 0) lengths[slot] = len + 1;
        else atomicOr(errw, static_cast<uint32_t>(SANDY_DEVERR_BLOCK));  // no page reserved for the row
    }
}

// one new grow row per tensor; position = device length; block per tensor
__global__ __launch_bounds__(256) void paged_append_step_kernel(const char* __restrict__ rows, char* __restrict__ pages,
                                                                const int32_t* __restrict__ table,
                                                                int32_t* __restrict__ lengths, int64_t max_blocks,
                                                                int64_t prefix, int64_t page_size, int64_t row_bytes,
                                                                int64_t page_bytes, uint32_t* errw, StepArgs args,
                                                                int32_t aligned16) {
    append_step_row(rows, pages, table, lengths, max_blocks, prefix, page_size, row_bytes, page_bytes, errw,
                    blockIdx.x, args.slots[blockIdx.x], aligned16);
}

// The K and V step appends of one decode step in one launch: blockIdx.y
// selects the set (0: K, 1: V), blockIdx.x the tensor.
constexpr int kMaxKvStep = 64;
struct KvStepSet {
    const char* rows;
    char* pages;
    const int32_t* table;
    int32_t* lengths;
    int64_t max_blocks, prefix, page_size, row_bytes, page_bytes;
    int32_t aligned16;
    int32_t slots[kMaxKvStep];
};

__global__ __launch_bounds__(256) void paged_append_step_kv_kernel(KvStepSet k, KvStepSet v, uint32_t* errw) {
    const KvStepSet& a = blockIdx.y ? v : k;
    append_step_row(a.rows, a.pages, a.table, a.lengths, a.max_blocks, a.prefix, a.page_size, a.row_bytes,
                    a.page_bytes, errw, blockIdx.x, a.slots[blockIdx.x], a.aligned16);
}

// One decode step's q/k/v post-processing for `count` sequences in one
// launch (workgroup b = sequence b): RoPE of the q heads into q_out, RoPE of
// the k heads appended as the next row of sequence b's K tensor, the v heads
// appended to its V tensor, both lengths advanced.  Same arithmetic as
// sandy_hip_rope (host powf denominators, correctly rounded angle, rope_sincos,
// bf16 round to nearest even) and the step append.
constexpr int kMaxFusedStep = 256;
constexpr int kMaxFusedPairs = 128;

struct DecodeQkvArgs {
    const uint16_t* qkv;
    int64_t row_stride;  // elements between sequences' qkv rows
    int32_t hq, hkv, d, split_half;
    const void* pos;
    int32_t pos_dt;
    uint16_t* q_out;     // [count, hq, d]
    char* k_pages;
    char* v_pages;
    const int32_t* k_table;
    const int32_t* v_table;
    int32_t* k_len;
    int32_t* v_len;
    int64_t k_max_blocks, v_max_blocks, page_size, page_bytes;
    uint32_t* errw;
    float denom[kMaxFusedPairs];
    int32_t k_slots[kMaxFusedStep];
    int32_t v_slots[kMaxFusedStep];
};

// STAGED (head_dim % 8 == 0, 16-byte aligned rows of at most 16 KiB): the
// position and lengths are requested first, then the sequence's whole q/k/v
// row as 16-byte pieces (up to four per thread in flight); the block-table
// reads that depend on the lengths go out while the row is still arriving.
// The rotation, the K append and the 16-byte V copy then read the row from
// LDS.  Otherwise each pair is read from global memory.
constexpr int kStageRowBytes = 16384;

template <bool STAGED>
__global__ __launch_bounds__(256) void decode_qkv_kernel(DecodeQkvArgs a) {
    __shared__ __attribute__((aligned(16))) uint16_t srow[STAGED ? kStageRowBytes / 2 : 8];
    __shared__ float sden[kMaxFusedPairs];
    const int b = blockIdx.x;
    const uint16_t* grow = a.qkv + b * a.row_stride;
    const int n = (a.hq + 2 * a.hkv) * a.d;
    const int nv = n / 8;  // 16-byte pieces of the row, at most 1024 when staged: four per thread
    const int t0 = threadIdx.x;
    const int v0 = t0 < nv ? t0 : nv - 1, v1 = t0 + 256 < nv ? t0 + 256 : nv - 1;
    const int v2 = t0 + 512 < nv ? t0 + 512 : nv - 1, v3 = t0 + 768 < nv ? t0 + 768 : nv - 1;
    uint4 p0{}, p1{}, p2{}, p3{};
    if constexpr (STAGED) {  // the row's loads go out first: they depend on nothing
        const uint4* g16 = reinterpret_cast<const uint4*>(grow);
        p0 = g16[v0];
        p1 = g16[v1];
        p2 = g16[v2];
        p3 = g16[v3];
    }
    // the angle denominators, indexed per lane, read once into LDS (a
    // per-lane index into the argument block is a memory load per use)
    const float den = a.denom[threadIdx.x < kMaxFusedPairs ? threadIdx.x : 0];
    __builtin_amdgcn_sched_barrier(0);  // keep those loads ahead of the slot -> length -> table chain
    const int32_t ks = a.k_slots[b], vs = a.v_slots[b];
    int64_t pos = load_index(a.pos, a.pos_dt, b);
    const int32_t kl = a.k_len[ks], vl = a.v_len[vs];
    const int32_t kblk = kl / a.page_size < a.k_max_blocks ? a.k_table[ks * a.k_max_blocks + kl / a.page_size] : -1;
    const int32_t vblk = vl / a.page_size < a.v_max_blocks ? a.v_table[vs * a.v_max_blocks + vl / a.page_size] : -1;
    if (threadIdx.x < kMaxFusedPairs) sden[threadIdx.x] = den;
    if constexpr (STAGED) {
        // unconditional stores (a guarded store would pull its load in behind
        // the guard); clamped pieces rewrite the same bytes
        uint4* s16 = reinterpret_cast<uint4*>(srow);
        s16[v0] = p0;
        s16[v1] = p1;
        s16[v2] = p2;
        s16[v3] = p3;
    }
    __syncthreads();  // the row is staged, and every thread has read the lengths before they advance
    if (pos < 0) {
        if (threadIdx.x == 0) atomicOr(a.errw, static_cast<uint32_t>(SANDY_DEVERR_POSITION));
        pos = 0;
    }
    const uint16_t* row = STAGED ? srow : grow;
    const int half = a.d >> 1;
    const float fp = static_cast<float>(pos);
    const int64_t row_bytes = static_cast<int64_t>(a.d) * 2;
    for (int pi = threadIdx.x; pi < (a.hq + a.hkv) * half; pi += 256) {
        const int head = pi / half, i = pi - head * half;
        const int i0 = a.split_half ? i : 2 * i, i1 = a.split_half ? i + half : 2 * i + 1;
        const float x0 = bf16_to_f32(row[head * a.d + i0]), x1 = bf16_to_f32(row[head * a.d + i1]);
        float sn, cs;
        rope_sincos(fp / sden[i], &sn, &cs);
        const uint16_t r0 = f32_to_bf16(__fsub_rn(__fmul_rn(x0, cs), __fmul_rn(x1, sn)));
        const uint16_t r1 = f32_to_bf16(__fadd_rn(__fmul_rn(x0, sn), __fmul_rn(x1, cs)));
        if (head < a.hq) {
            uint16_t* q = a.q_out + (static_cast<int64_t>(b) * a.hq + head) * a.d;
            q[i0] = r0;
            q[i1] = r1;
        } else if (kblk >= 0) {
            uint16_t* kd = reinterpret_cast<uint16_t*>(
                a.k_pages + kblk * a.page_bytes + ((head - a.hq) * a.page_size + kl % a.page_size) * row_bytes);
            kd[i0] = r0;
            kd[i1] = r1;
        }
    }
    if (vblk >= 0) {
        const uint16_t* v = row + (a.hq + a.hkv) * a.d;
        if constexpr (STAGED) {
            for (int e8 = threadIdx.x; e8 < a.hkv * a.d / 8; e8 += 256) {
                const int e = e8 * 8, kh = e / a.d;
                char* vd = a.v_pages + vblk * a.page_bytes + (kh * a.page_size + vl % a.page_size) * row_bytes +
                           static_cast<int64_t>(e - kh * a.d) * 2;
                *reinterpret_cast<uint4*>(vd) = *reinterpret_cast<const uint4*>(v + e);
            }
        } else {
            for (int e = threadIdx.x; e < a.hkv * a.d; e += 256) {
                const int kh = e / a.d;
                uint16_t* vd = reinterpret_cast<uint16_t*>(
                    a.v_pages + vblk * a.page_bytes + (kh * a.page_size + vl % a.page_size) * row_bytes);
                vd[e - kh * a.d] = v[e];
            }
        }
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        if (kblk >= 0) a.k_len[ks] = kl + 1;
        if (vblk >= 0) a.v_len[vs] = vl + 1;
        if (kblk < 0 || vblk < 0) atomicOr(a.errw, static_cast<uint32_t>(SANDY_DEVERR_BLOCK));  // no page reserved
    }
}

__global__ void paged_positions_kernel(const int32_t* __restrict__ lengths, void* __restrict__ out, int32_t out_dt,
                                       int32_t count, int32_t delta, StepArgs args) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < count) store_index(out, out_dt, i, static_cast<int64_t>(lengths[args.slots[i]]) + delta);
}

} // namespace

struct HipDeviceImpl {
    int ordinal = 0;
    hipStream_t stream = nullptr;
    uint32_t next_id = 1;
    std::map<uint32_t, std::pair<void*, size_t>> buffers;
    std::map<uint32_t, std::unique_ptr<PagedPool>> pools;
    std::map<uint32_t, PagedTensor> tensors;
    std::map<uint32_t, hipGraphExec_t> graphs;
    hipGraph_t capturing = nullptr;
    std::mutex mu;
};

} // namespace sandy_hip

struct SandyHipDevice {
    sandy_hip::HipDeviceImpl impl;
};

using namespace sandy_hip;

namespace {

int set_device(SandyHipDevice* d, Err e) {
    if (!d) return fail(e, SANDY_ERR_INVALID, "hip device is null");
    SANDY_HIP_TRY(hipSetDevice(d->impl.ordinal), e, "hipSetDevice");
    return SANDY_OK;
}

int64_t product(const int64_t* dims, int lo, int hi) {
    int64_t p = 1;
    for (int i = lo; i < hi; i++) p *= dims[i];
    return p;
}

// CudaPagedTensor.cpp:30-55 validate_paged_pool_desc, Device.cpp:13-19
int validate_pool(const SandyPagedPoolDesc& d, Err e) {
    if (d.rank <= 0 || d.rank > SANDY_HIP_MAX_RANK) return fail(e, SANDY_ERR_INVALID, "paged tensor pool rank must be >= 1");
    if (d.grow_dim < 0 || d.grow_dim >= d.rank) return fail(e, SANDY_ERR_INVALID, "paged tensor pool grow_dim out of range");
    if (d.page_size <= 0) return fail(e, SANDY_ERR_INVALID, "paged tensor pool page_size must be > 0");
    if ((d.page_size & (d.page_size - 1)) != 0)
        return fail(e, SANDY_ERR_INVALID, "paged tensor pool page_size must be a power of two");
    if (d.initial_pages < 0) return fail(e, SANDY_ERR_INVALID, "paged tensor pool initial page count must be >= 0");
    if (d.max_pages >= 0 && d.initial_pages > d.max_pages)
        return fail(e, SANDY_ERR_INVALID, "paged tensor pool initial page count exceeds max page count");
    for (int i = 0; i < d.rank; i++)
        if (i != d.grow_dim && d.dims[i] <= 0)
            return fail(e, SANDY_ERR_INVALID, "paged tensor pool non-grow dimensions must be static and positive");
    if (!is_float(d.dtype) && d.dtype != SANDY_I32 && d.dtype != SANDY_I64)
        return fail(e, SANDY_ERR_INVALID, "paged tensor pool unsupported dtype");
    if (d.max_tensors <= 0 || d.max_blocks <= 0)
        return fail(e, SANDY_ERR_INVALID, "paged tensor pool needs max_tensors and max_blocks > 0");
    return SANDY_OK;
}

// Grows the page allocation to hold at least `need` pages (doubling).  Any
// captured graph that used the old allocation must be re-captured.
int grow_pool(HipDeviceImpl& d, PagedPool& p, int64_t need, Err e) {
    if (need <= p.capacity) return SANDY_OK;
    if (p.desc.max_pages >= 0 && need > p.desc.max_pages)
        return fail(e, SANDY_ERR_INVALID, "hip device paged pool capacity exceeded");
    int64_t cap = std::max<int64_t>(need, std::max<int64_t>(16, 2 * p.capacity));
    if (p.desc.max_pages >= 0) cap = std::min(cap, p.desc.max_pages);
    char* fresh = nullptr;
    SANDY_HIP_TRY(hipMalloc(reinterpret_cast<void**>(&fresh), static_cast<size_t>(cap * p.page_elems) * p.elem), e,
                  "paged pool allocation");
    if (p.pages) {
        SANDY_HIP_TRY(hipMemcpyAsync(fresh, p.pages, static_cast<size_t>(p.capacity * p.page_elems) * p.elem,
                                     hipMemcpyDeviceToDevice, d.stream), e, "paged pool growth copy");
        SANDY_HIP_TRY(hipStreamSynchronize(d.stream), e, "paged pool growth");
        SANDY_HIP_TRY(hipFree(p.pages), e, "paged pool release");
    }
    p.pages = fresh;
    p.capacity = cap;
    return SANDY_OK;
}

int take_page(HipDeviceImpl& d, PagedPool& p, int32_t* page, Err e) {
    if (!p.free_pages.empty()) {
        *page = p.free_pages.back();
        p.free_pages.pop_back();
        return SANDY_OK;
    }
    if (p.used >= 0x7fffffff) return fail(e, SANDY_ERR_INVALID, "hip device paged pool page index overflow");
    int st = grow_pool(d, p, p.used + 1, e);
    if (st) return st;
    *page = static_cast<int32_t>(p.used++);
    return SANDY_OK;
}

// CpuDevice.cpp:444-463 reservePaged: append pages until page_count; the new
// block-table entries are copied to the device on the stream.
int reserve(HipDeviceImpl& d, PagedTensor& t, int64_t page_count, Err e) {
    if (page_count < 0) return fail(e, SANDY_ERR_INVALID, "hip device paged tensor reserve page count must be >= 0");
    PagedPool& p = *d.pools.at(t.pool);
    if (page_count > p.desc.max_blocks)
        return fail(e, SANDY_ERR_INVALID, "hip device paged tensor exceeds the pool's max_blocks");
    const size_t first = t.pages.size();
    while (static_cast<int64_t>(t.pages.size()) < page_count) {
        int32_t page = 0;
        int st = take_page(d, p, &page, e);
        if (st) return st;
        t.pages.push_back(page);
    }
    if (t.pages.size() > first) {
        const size_t n = t.pages.size() - first;
        // entries go through the pinned mirror, which stays valid until the copy runs
        int32_t* src = p.host_table + static_cast<int64_t>(t.slot) * p.desc.max_blocks + first;
        std::copy(t.pages.begin() + static_cast<std::ptrdiff_t>(first), t.pages.end(), src);
        SANDY_HIP_TRY(hipMemcpyAsync(p.table + t.slot * p.desc.max_blocks + first, src, n * sizeof(int32_t),
                                     hipMemcpyHostToDevice, d.stream), e, "block table update");
    }
    return SANDY_OK;
}

} // namespace

extern "C" {

int sandy_hip_device_create(int32_t ordinal, SandyHipDevice** out, char* err, size_t err_cap) {
    Err e{err, err_cap};
    if (!out) return fail(e, SANDY_ERR_INVALID, "hip device output pointer is null");
    int count = 0;
    SANDY_HIP_TRY(hipGetDeviceCount(&count), e, "hipGetDeviceCount");
    if (ordinal < 0 || ordinal >= count) return fail(e, SANDY_ERR_INVALID, "hip device ordinal %d out of range", ordinal);
    auto* d = new SandyHipDevice();
    d->impl.ordinal = ordinal;
    hipError_t st = hipSetDevice(ordinal);
    if (st == hipSuccess) st = hipStreamCreateWithFlags(&d->impl.stream, hipStreamNonBlocking);
    if (st != hipSuccess) {
        delete d;
        return fail(e, SANDY_ERR_HIP, "hip device stream: %s", hipGetErrorString(st));
    }
    *out = d;
    return ok(e);
}

void sandy_hip_device_destroy(SandyHipDevice* d) {
    if (!d) return;
    auto& m = d->impl;
    hipSetDevice(m.ordinal);
    hipStreamSynchronize(m.stream);
    for (auto& g : m.graphs) hipGraphExecDestroy(g.second);
    for (auto& b : m.buffers) hipFree(b.second.first);
    for (auto& p : m.pools) {
        hipFree(p.second->pages);
        hipFree(p.second->table);
        hipFree(p.second->lengths);
        hipHostFree(p.second->host_table);
    }
    hipStreamDestroy(m.stream);
    delete d;
}

void* sandy_hip_device_stream(SandyHipDevice* d) { return d ? d->impl.stream : nullptr; }

int sandy_hip_device_synchronize(SandyHipDevice* d, char* err, size_t err_cap) {
    Err e{err, err_cap};
    int st = set_device(d, e);
    if (st) return st;
    SANDY_HIP_TRY(hipStreamSynchronize(d->impl.stream), e, "hipStreamSynchronize");
    return ok(e);
}

int sandy_hip_device_alloc(SandyHipDevice* d, uint64_t bytes, uint32_t* buffer, char* err, size_t err_cap) {
    Err e{err, err_cap};
    int st = set_device(d, e);
    if (st) return st;
    if (d->impl.capturing) return fail(e, SANDY_ERR_INVALID, "%s is not allowed during graph capture", __func__);
    std::lock_guard<std::mutex> lock(d->impl.mu);
    void* p = nullptr;
    SANDY_HIP_TRY(hipMalloc(&p, bytes ? bytes : 16), e, "hip device alloc");
    const uint32_t id = d->impl.next_id++;
    d->impl.buffers[id] = {p, bytes};
    *buffer = id;
    return ok(e);
}

int sandy_hip_device_dealloc(SandyHipDevice* d, uint32_t buffer, char* err, size_t err_cap) {
    Err e{err, err_cap};
    int st = set_device(d, e);
    if (st) return st;
    if (d->impl.capturing) return fail(e, SANDY_ERR_INVALID, "%s is not allowed during graph capture", __func__);
    std::lock_guard<std::mutex> lock(d->impl.mu);
    auto it = d->impl.buffers.find(buffer);
    if (it == d->impl.buffers.end()) return fail(e, SANDY_ERR_INVALID, "hip device buffer not found");
    SANDY_HIP_TRY(hipStreamSynchronize(d->impl.stream), e, "hipStreamSynchronize");
    SANDY_HIP_TRY(hipFree(it->second.first), e, "hip device dealloc");
    d->impl.buffers.erase(it);
    return ok(e);
}

void* sandy_hip_device_buffer(SandyHipDevice* d, uint32_t buffer) {
    if (!d) return nullptr;
    std::lock_guard<std::mutex> lock(d->impl.mu);
    auto it = d->impl.buffers.find(buffer);
    return it == d->impl.buffers.end() ? nullptr : it->second.first;
}

int sandy_hip_device_load(SandyHipDevice* d, const void* host, uint64_t bytes, uint32_t* buffer, char* err,
                          size_t err_cap) {
    Err e{err, err_cap};
    int st = sandy_hip_device_alloc(d, bytes, buffer, err, err_cap);
    if (st) return st;
    void* p = sandy_hip_device_buffer(d, *buffer);
    SANDY_HIP_TRY(hipMemcpyAsync(p, host, bytes, hipMemcpyHostToDevice, d->impl.stream), e, "hip device load");
    SANDY_HIP_TRY(hipStreamSynchronize(d->impl.stream), e, "hip device load");
    return ok(e);
}

int sandy_hip_device_read(SandyHipDevice* d, uint32_t buffer, uint64_t offset, uint64_t bytes, void* host, char* err,
                          size_t err_cap) {
    Err e{err, err_cap};
    int st = set_device(d, e);
    if (st) return st;
    void* p = nullptr;
    {
        std::lock_guard<std::mutex> lock(d->impl.mu);
        auto it = d->impl.buffers.find(buffer);
        if (it == d->impl.buffers.end()) return fail(e, SANDY_ERR_INVALID, "hip device buffer not found");
        if (offset + bytes > it->second.second) return fail(e, SANDY_ERR_INVALID, "hip device read exceeds the buffer");
        p = static_cast<char*>(it->second.first) + offset;
    }
    SANDY_HIP_TRY(hipMemcpyAsync(host, p, bytes, hipMemcpyDeviceToHost, d->impl.stream), e, "hip device read");
    SANDY_HIP_TRY(hipStreamSynchronize(d->impl.stream), e, "hip device read");
    return ok(e);
}

int sandy_hip_device_paged_pool_create(SandyHipDevice* d, const SandyPagedPoolDesc* desc, uint32_t* pool, char* err,
                                       size_t err_cap) {
    Err e{err, err_cap};
    int st = set_device(d, e);
    if (st) return st;
    if (d->impl.capturing) return fail(e, SANDY_ERR_INVALID, "%s is not allowed during graph capture", __func__);
    if (!desc || !pool) return fail(e, SANDY_ERR_INVALID, "paged pool descriptor is null");
    st = validate_pool(*desc, e);
    if (st) return st;
    std::lock_guard<std::mutex> lock(d->impl.mu);
    auto p = std::make_unique<PagedPool>();
    p->desc = *desc;
    p->prefix = product(desc->dims, 0, static_cast<int>(desc->grow_dim));
    p->inner = product(desc->dims, static_cast<int>(desc->grow_dim) + 1, desc->rank);
    p->page_elems = p->prefix * desc->page_size * p->inner;
    p->elem = dtype_size(desc->dtype);
    SANDY_HIP_TRY(hipMalloc(reinterpret_cast<void**>(&p->table), static_cast<size_t>(desc->max_tensors * desc->max_blocks) * 4),
                  e, "block table allocation");
    SANDY_HIP_TRY(hipMalloc(reinterpret_cast<void**>(&p->lengths), static_cast<size_t>(desc->max_tensors) * 4), e,
                  "length allocation");
    SANDY_HIP_TRY(hipHostMalloc(reinterpret_cast<void**>(&p->host_table),
                                static_cast<size_t>(desc->max_tensors * desc->max_blocks) * 4, hipHostMallocDefault),
                  e, "pinned block table mirror");
    SANDY_HIP_TRY(hipMemsetAsync(p->table, 0xff, static_cast<size_t>(desc->max_tensors * desc->max_blocks) * 4, d->impl.stream),
                  e, "block table init");
    SANDY_HIP_TRY(hipMemsetAsync(p->lengths, 0, static_cast<size_t>(desc->max_tensors) * 4, d->impl.stream), e, "length init");
    st = grow_pool(d->impl, *p, std::max<int64_t>(1, desc->initial_pages), e);
    if (st) return st;
    for (int64_t s = desc->max_tensors - 1; s >= 0; s--) p->free_slots.push_back(static_cast<int32_t>(s));
    SANDY_HIP_TRY(hipStreamSynchronize(d->impl.stream), e, "paged pool create");
    const uint32_t id = d->impl.next_id++;
    d->impl.pools[id] = std::move(p);
    *pool = id;
    return ok(e);
}

int sandy_hip_device_paged_pool_destroy(SandyHipDevice* d, uint32_t pool, char* err, size_t err_cap) {
    Err e{err, err_cap};
    int st = set_device(d, e);
    if (st) return st;
    std::lock_guard<std::mutex> lock(d->impl.mu);
    auto it = d->impl.pools.find(pool);
    if (it == d->impl.pools.end()) return fail(e, SANDY_ERR_INVALID, "hip device paged pool not found");
    for (auto& t : d->impl.tensors)
        if (t.second.pool == pool) return fail(e, SANDY_ERR_INVALID, "hip device paged pool still has tensors");
    SANDY_HIP_TRY(hipStreamSynchronize(d->impl.stream), e, "hipStreamSynchronize");
    hipFree(it->second->pages);
    hipFree(it->second->table);
    hipFree(it->second->lengths);
    hipHostFree(it->second->host_table);
    d->impl.pools.erase(it);
    return ok(e);
}

int sandy_hip_device_paged_alloc(SandyHipDevice* d, uint32_t pool, uint32_t* tensor, char* err, size_t err_cap) {
    Err e{err, err_cap};
    int st = set_device(d, e);
    if (st) return st;
    if (d->impl.capturing) return fail(e, SANDY_ERR_INVALID, "%s is not allowed during graph capture", __func__);
    std::lock_guard<std::mutex> lock(d->impl.mu);
    auto it = d->impl.pools.find(pool);
    if (it == d->impl.pools.end()) return fail(e, SANDY_ERR_INVALID, "hip device paged pool not found");
    PagedPool& p = *it->second;
    if (p.free_slots.empty()) return fail(e, SANDY_ERR_INVALID, "hip device paged pool has no free tensor slot");
    PagedTensor t;
    t.pool = pool;
    t.slot = p.free_slots.back();
    p.free_slots.pop_back();
    SANDY_HIP_TRY(hipMemsetAsync(p.lengths + t.slot, 0, 4, d->impl.stream), e, "length reset");
    const uint32_t id = d->impl.next_id++;
    d->impl.tensors[id] = std::move(t);
    *tensor = id;
    return ok(e);
}

int sandy_hip_device_paged_dealloc(SandyHipDevice* d, uint32_t tensor, char* err, size_t err_cap) {
    Err e{err, err_cap};
    int st = set_device(d, e);
    if (st) return st;
    if (d->impl.capturing) return fail(e, SANDY_ERR_INVALID, "%s is not allowed during graph capture", __func__);
    std::lock_guard<std::mutex> lock(d->impl.mu);
    auto it = d->impl.tensors.find(tensor);
    if (it == d->impl.tensors.end()) return fail(e, SANDY_ERR_INVALID, "hip device paged tensor not found");
    PagedPool& p = *d->impl.pools.at(it->second.pool);
    for (int32_t page : it->second.pages) p.free_pages.push_back(page);  // pages return to the free list
    SANDY_HIP_TRY(hipMemsetAsync(p.table + it->second.slot * p.desc.max_blocks, 0xff,
                                 static_cast<size_t>(p.desc.max_blocks) * 4, d->impl.stream), e, "block table reset");
    p.free_slots.push_back(it->second.slot);
    d->impl.tensors.erase(it);
    return ok(e);
}

int sandy_hip_device_paged_reserve(SandyHipDevice* d, uint32_t tensor, int64_t page_count, char* err, size_t err_cap) {
    Err e{err, err_cap};
    int st = set_device(d, e);
    if (st) return st;
    if (d->impl.capturing) return fail(e, SANDY_ERR_INVALID, "%s is not allowed during graph capture", __func__);
    std::lock_guard<std::mutex> lock(d->impl.mu);
    auto it = d->impl.tensors.find(tensor);
    if (it == d->impl.tensors.end()) return fail(e, SANDY_ERR_INVALID, "hip device paged tensor not found");
    st = reserve(d->impl, it->second, page_count, e);
    return st ? st : ok(e);
}

int sandy_hip_device_paged_append(SandyHipDevice* d, uint32_t tensor, const SandyTensor* chunk, char* err,
                                  size_t err_cap) {
    Err e{err, err_cap};
    int st = set_device(d, e);
    if (st) return st;
    if (d->impl.capturing) return fail(e, SANDY_ERR_INVALID, "%s is not allowed during graph capture", __func__);
    std::lock_guard<std::mutex> lock(d->impl.mu);
    auto it = d->impl.tensors.find(tensor);
    if (it == d->impl.tensors.end()) return fail(e, SANDY_ERR_INVALID, "hip device paged tensor not found");
    PagedTensor& t = it->second;
    PagedPool& p = *d->impl.pools.at(t.pool);
    if (!chunk || chunk->rank != p.desc.rank) return fail(e, SANDY_ERR_INVALID, "hip device paged append chunk rank mismatch");
    for (int i = 0; i < p.desc.rank; i++)
        if (i != p.desc.grow_dim && chunk->dims[i] != p.desc.dims[i])
            return fail(e, SANDY_ERR_INVALID, "hip device paged append chunk shape mismatch");
    if (chunk->dtype != p.desc.dtype) return fail(e, SANDY_ERR_INVALID, "hip device paged append dtype mismatch");
    if (!contiguous(*chunk)) return fail(e, SANDY_ERR_INVALID, "hip device paged append requires a contiguous source view");
    const int64_t chunk_len = chunk->dims[p.desc.grow_dim];
    if (chunk_len <= 0) return fail(e, SANDY_ERR_INVALID, "hip device paged append grow dimension must be > 0");
    const int64_t new_len = t.grow_length + chunk_len;
    st = reserve(d->impl, t, (new_len + p.desc.page_size - 1) / p.desc.page_size, e);
    if (st) return st;
    const int64_t rows = p.prefix * chunk_len;
    hipLaunchKernelGGL(paged_append_kernel, dim3(static_cast<unsigned>((rows + 3) / 4)), dim3(256), 0, d->impl.stream,
                       static_cast<const char*>(base_ptr(*chunk)), p.pages, p.table + t.slot * p.desc.max_blocks,
                       p.lengths + t.slot, t.grow_length, chunk_len, p.prefix, p.desc.page_size,
                       static_cast<int64_t>(p.inner * p.elem), static_cast<int64_t>(p.page_elems * p.elem));
    SANDY_HIP_TRY(hipGetLastError(), e, "paged append launch");
    t.grow_length = new_len;
    return ok(e);
}

int sandy_hip_device_paged_append_step(SandyHipDevice* d, uint32_t pool, const uint32_t* tensors, int32_t count,
                                       const SandyTensor* rows, char* err, size_t err_cap) {
    Err e{err, err_cap};
    int st = set_device(d, e);
    if (st) return st;
    std::lock_guard<std::mutex> lock(d->impl.mu);
    auto pit = d->impl.pools.find(pool);
    if (pit == d->impl.pools.end()) return fail(e, SANDY_ERR_INVALID, "hip device paged pool not found");
    PagedPool& p = *pit->second;
    if (count <= 0 || count > kMaxStepTensors) return fail(e, SANDY_ERR_INVALID, "paged append step count out of range");
    if (!rows || !contiguous(*rows) || rows->dtype != p.desc.dtype || numel(*rows) != count * p.prefix * p.inner)
        return fail(e, SANDY_ERR_INVALID, "hip device paged append step rows shape mismatch");
    uint32_t* errw = device_error_word(e, &st);
    if (st) return st;
    StepArgs args{};
    for (int i = 0; i < count; i++) {
        auto it = d->impl.tensors.find(tensors[i]);
        if (it == d->impl.tensors.end() || it->second.pool != pool)
            return fail(e, SANDY_ERR_INVALID, "hip device paged tensor not found");
        // two rows for one tensor would race on its device length
        for (int j = 0; j < i; j++)
            if (tensors[j] == tensors[i])
                return fail(e, SANDY_ERR_INVALID, "paged append step tensors must be distinct");
    }
    for (int i = 0; i < count; i++) {
        auto it = d->impl.tensors.find(tensors[i]);
        PagedTensor& t = it->second;
        // host bookkeeping advances in step with the device (graph replays: see paged_sync)
        if (t.grow_length + 1 > static_cast<int64_t>(t.pages.size()) * p.desc.page_size && !d->impl.capturing) {
            st = reserve(d->impl, t, (t.grow_length + p.desc.page_size) / p.desc.page_size, e);
            if (st) return st;
        }
        t.grow_length += 1;
        args.slots[i] = t.slot;
    }
    hipLaunchKernelGGL(paged_append_step_kernel, dim3(static_cast<unsigned>(count)), dim3(256), 0, d->impl.stream,
                       static_cast<const char*>(base_ptr(*rows)), p.pages, p.table, p.lengths, p.desc.max_blocks,
                       p.prefix, p.desc.page_size, static_cast<int64_t>(p.inner * p.elem),
                       static_cast<int64_t>(p.page_elems * p.elem), errw, args,
                       static_cast<int32_t>(((reinterpret_cast<uintptr_t>(base_ptr(*rows)) |
                                              reinterpret_cast<uintptr_t>(p.pages)) & 15u) == 0));
    SANDY_HIP_TRY(hipGetLastError(), e, "paged append step launch");
    return ok(e);
}

int sandy_hip_device_paged_append_step_kv(SandyHipDevice* d, uint32_t k_pool, const uint32_t* k_tensors,
                                          uint32_t v_pool, const uint32_t* v_tensors, int32_t count,
                                          const SandyTensor* k_rows, const SandyTensor* v_rows, char* err,
                                          size_t err_cap) {
    Err e{err, err_cap};
    int st = set_device(d, e);
    if (st) return st;
    std::lock_guard<std::mutex> lock(d->impl.mu);
    if (count <= 0 || count > kMaxKvStep)
        return fail(e, SANDY_ERR_INVALID, "paged append step count out of range (K and V together: at most %d)", kMaxKvStep);
    if (!k_tensors || !v_tensors) return fail(e, SANDY_ERR_INVALID, "hip device paged tensor not found");
    const uint32_t pools[2] = {k_pool, v_pool};
    const uint32_t* ids[2] = {k_tensors, v_tensors};
    const SandyTensor* rows[2] = {k_rows, v_rows};
    PagedPool* pp[2] = {nullptr, nullptr};
    // every check before any bookkeeping moves
    for (int s = 0; s < 2; s++) {
        auto pit = d->impl.pools.find(pools[s]);
        if (pit == d->impl.pools.end()) return fail(e, SANDY_ERR_INVALID, "hip device paged pool not found");
        pp[s] = pit->second.get();
        const PagedPool& p = *pp[s];
        if (!rows[s] || !contiguous(*rows[s]) || rows[s]->dtype != p.desc.dtype ||
            numel(*rows[s]) != count * p.prefix * p.inner)
            return fail(e, SANDY_ERR_INVALID, "hip device paged append step rows shape mismatch");
        for (int i = 0; i < count; i++) {
            auto it = d->impl.tensors.find(ids[s][i]);
            if (it == d->impl.tensors.end() || it->second.pool != pools[s])
                return fail(e, SANDY_ERR_INVALID, "hip device paged tensor not found");
            for (int j = 0; j < i; j++)
                if (ids[s][j] == ids[s][i]) return fail(e, SANDY_ERR_INVALID, "paged append step tensors must be distinct");
        }
    }
    if (k_pool == v_pool)
        for (int i = 0; i < count; i++)
            for (int j = 0; j < count; j++)
                if (k_tensors[i] == v_tensors[j])
                    return fail(e, SANDY_ERR_INVALID, "paged append step tensors must be distinct");
    uint32_t* errw = device_error_word(e, &st);
    if (st) return st;
    // pages for every new row first (outside capture), then the lengths
    for (int s = 0; s < 2; s++)
        for (int i = 0; i < count; i++) {
            PagedTensor& t = d->impl.tensors.at(ids[s][i]);
            const PagedPool& p = *pp[s];
            if (t.grow_length + 1 > static_cast<int64_t>(t.pages.size()) * p.desc.page_size && !d->impl.capturing) {
                st = reserve(d->impl, t, (t.grow_length + p.desc.page_size) / p.desc.page_size, e);
                if (st) return st;
            }
        }
    KvStepSet set[2];
    for (int s = 0; s < 2; s++) {
        const PagedPool& p = *pp[s];
        KvStepSet& a = set[s];
        a.rows = static_cast<const char*>(base_ptr(*rows[s]));
        a.pages = p.pages;
        a.table = p.table;
        a.lengths = p.lengths;
        a.max_blocks = p.desc.max_blocks;
        a.prefix = p.prefix;
        a.page_size = p.desc.page_size;
        a.row_bytes = static_cast<int64_t>(p.inner * p.elem);
        a.page_bytes = static_cast<int64_t>(p.page_elems * p.elem);
        a.aligned16 = static_cast<int32_t>(((reinterpret_cast<uintptr_t>(a.rows) | reinterpret_cast<uintptr_t>(p.pages)) & 15u) == 0);
        for (int i = 0; i < count; i++) {
            PagedTensor& t = d->impl.tensors.at(ids[s][i]);
            t.grow_length += 1;  // host bookkeeping in step with the device
            a.slots[i] = t.slot;
        }
    }
    hipLaunchKernelGGL(paged_append_step_kv_kernel, dim3(static_cast<unsigned>(count), 2), dim3(256), 0, d->impl.stream,
                       set[0], set[1], errw);
    SANDY_HIP_TRY(hipGetLastError(), e, "paged append step launch");
    return ok(e);
}

namespace {
// Shared set-up of the fused decode q/k/v entry points: the pools' geometry
// and the head counts checked, each sequence's K and V slot looked up, and
// the host bookkeeping advanced by one row (pages reserved outside capture),
// as for the step append.
struct QkvStep {
    PagedPool* kp = nullptr;
    PagedPool* vp = nullptr;
    int64_t hkv = 0, D = 0;
    int32_t k_slots[kMaxFusedStep];
    int32_t v_slots[kMaxFusedStep];
};

int qkv_step(SandyHipDevice* d, uint32_t k_pool, const uint32_t* k_tensors, uint32_t v_pool,
             const uint32_t* v_tensors, int32_t count, int32_t q_heads, const SandyTensor* positions, double theta,
             const SandyTensor* q_out, QkvStep& q, Err e) {
    auto kit = d->impl.pools.find(k_pool), vit = d->impl.pools.find(v_pool);
    if (kit == d->impl.pools.end() || vit == d->impl.pools.end())
        return fail(e, SANDY_ERR_INVALID, "hip device paged pool not found");
    PagedPool& kp = *kit->second;
    PagedPool& vp = *vit->second;
    if (count <= 0 || count > kMaxFusedStep) return fail(e, SANDY_ERR_INVALID, "decode qkv count out of range");
    if (kp.desc.dtype != SANDY_BF16 || vp.desc.dtype != SANDY_BF16 || kp.prefix != vp.prefix || kp.inner != vp.inner ||
        kp.desc.page_size != vp.desc.page_size)
        return fail(e, SANDY_ERR_INVALID, "decode qkv needs bf16 K and V pools of one geometry");
    const int64_t hkv = kp.prefix, D = kp.inner;
    if (D % 2 != 0 || D / 2 > kMaxFusedPairs) return fail(e, SANDY_ERR_UNSUPPORTED, "decode qkv head dimension unsupported");
    if (q_heads <= 0 || q_heads % hkv != 0) return fail(e, SANDY_ERR_INVALID, "attention heads must be divisible by kv_heads");
    if (!q_out || q_out->dtype != SANDY_BF16 || numel(*q_out) != count * q_heads * D || !contiguous(*q_out))
        return fail(e, SANDY_ERR_INVALID, "decode qkv q output must be contiguous [count, q_heads, 1, head_dim] bf16");
    if (!positions || !is_index(positions->dtype) || numel(*positions) != count || !contiguous(*positions))
        return fail(e, SANDY_ERR_INVALID, "rope position_ids numel must match the sequence count");
    if (static_cast<float>(theta) <= 0.0f) return fail(e, SANDY_ERR_INVALID, "rope theta must be > 0");
    // every id checked before any bookkeeping moves; two sequences naming one
    // tensor would write one row and advance its host length twice
    for (int i = 0; i < count; i++)
        for (int which = 0; which < 2; which++) {
            const uint32_t* ids = which ? v_tensors : k_tensors;
            auto it = d->impl.tensors.find(ids[i]);
            if (it == d->impl.tensors.end() || it->second.pool != (which ? v_pool : k_pool))
                return fail(e, SANDY_ERR_INVALID, "hip device paged tensor not found");
            for (int j = 0; j < i; j++)
                if (ids[j] == ids[i]) return fail(e, SANDY_ERR_INVALID, "decode qkv tensors must be distinct");
        }
    // pages first, for every tensor, so a failed reservation leaves no length
    // advanced; then the host bookkeeping advances in step with the device, as
    // for the step append
    for (int i = 0; i < count; i++)
        for (int which = 0; which < 2; which++) {
            PagedTensor& t = d->impl.tensors.find(which ? v_tensors[i] : k_tensors[i])->second;
            PagedPool& p = which ? vp : kp;
            if (t.grow_length + 1 > static_cast<int64_t>(t.pages.size()) * p.desc.page_size && !d->impl.capturing) {
                const int st = reserve(d->impl, t, (t.grow_length + p.desc.page_size) / p.desc.page_size, e);
                if (st) return st;
            }
        }
    for (int i = 0; i < count; i++) {
        for (int which = 0; which < 2; which++) {
            PagedTensor& t = d->impl.tensors.find(which ? v_tensors[i] : k_tensors[i])->second;
            t.grow_length += 1;
            (which ? q.v_slots : q.k_slots)[i] = t.slot;
        }
    }
    q.kp = &kp;
    q.vp = &vp;
    q.hkv = hkv;
    q.D = D;
    return SANDY_OK;
}
} // namespace

int sandy_hip_device_decode_qkv(SandyHipDevice* d, uint32_t k_pool, const uint32_t* k_tensors, uint32_t v_pool,
                                const uint32_t* v_tensors, int32_t count, const SandyTensor* qkv, int32_t q_heads,
                                const SandyTensor* positions, double theta, int32_t split_half,
                                const SandyTensor* q_out, char* err, size_t err_cap) {
    Err e{err, err_cap};
    int st = set_device(d, e);
    if (st) return st;
    std::lock_guard<std::mutex> lock(d->impl.mu);
    auto kit = d->impl.pools.find(k_pool);
    if (kit != d->impl.pools.end() && kit->second->prefix > 0) {
        const int64_t hkv = kit->second->prefix, D = kit->second->inner;
        if (q_heads <= 0 || q_heads % hkv != 0)
            return fail(e, SANDY_ERR_INVALID, "attention heads must be divisible by kv_heads");
        if (!qkv || qkv->dtype != SANDY_BF16 || qkv->rank != 2 || qkv->dims[0] != count ||
            qkv->dims[1] != (q_heads + 2 * hkv) * D || qkv->strides[1] != 1)
            return fail(e, SANDY_ERR_INVALID, "decode qkv input must be [count, (q_heads + 2 kv_heads) head_dim] bf16");
    }
    uint32_t* errw = device_error_word(e, &st);
    if (st) return st;
    QkvStep q;
    st = qkv_step(d, k_pool, k_tensors, v_pool, v_tensors, count, q_heads, positions, theta, q_out, q, e);
    if (st) return st;
    PagedPool& kp = *q.kp;
    PagedPool& vp = *q.vp;
    const int64_t hkv = q.hkv, D = q.D;
    const float th = static_cast<float>(theta);
    DecodeQkvArgs a{};
    std::copy(q.k_slots, q.k_slots + count, a.k_slots);
    std::copy(q.v_slots, q.v_slots + count, a.v_slots);
    a.qkv = static_cast<const uint16_t*>(base_ptr(*qkv));
    a.row_stride = qkv->strides[0];
    a.hq = q_heads;
    a.hkv = static_cast<int32_t>(hkv);
    a.d = static_cast<int32_t>(D);
    a.split_half = split_half ? 1 : 0;
    a.pos = base_ptr(*positions);
    a.pos_dt = positions->dtype;
    a.q_out = static_cast<uint16_t*>(base_ptr(*q_out));
    a.k_pages = kp.pages;
    a.v_pages = vp.pages;
    a.k_table = kp.table;
    a.v_table = vp.table;
    a.k_len = kp.lengths;
    a.v_len = vp.lengths;
    a.k_max_blocks = kp.desc.max_blocks;
    a.v_max_blocks = vp.desc.max_blocks;
    a.page_size = kp.desc.page_size;
    a.page_bytes = static_cast<int64_t>(kp.page_elems * kp.elem);
    a.errw = errw;
    // the rope kernel's denominators: theta^(2i/d) in float, as the CPU reference
    for (int i = 0; i < D / 2; i++) a.denom[i] = std::pow(th, static_cast<float>(2 * i) / static_cast<float>(D));
    const bool staged = D % 8 == 0 && a.row_stride % 8 == 0 && (reinterpret_cast<uintptr_t>(a.qkv) & 15) == 0 &&
                        (q_heads + 2 * hkv) * D * 2 <= kStageRowBytes;
    if (staged) hipLaunchKernelGGL(decode_qkv_kernel<true>, dim3(static_cast<unsigned>(count)), dim3(256), 0, d->impl.stream, a);
    else hipLaunchKernelGGL(decode_qkv_kernel<false>, dim3(static_cast<unsigned>(count)), dim3(256), 0, d->impl.stream, a);
    SANDY_HIP_TRY(hipGetLastError(), e, "decode qkv launch");
    return ok(e);
}

int sandy_hip_device_matmul_qkv(SandyHipDevice* d, const SandyTensor* lhs, const SandyRowStats* lhs_stats,
                                const SandyTensor* norm_weight, double eps, const SandyTensor* rhs, uint32_t k_pool,
                                const uint32_t* k_tensors, uint32_t v_pool, const uint32_t* v_tensors, int32_t count,
                                int32_t q_heads, const SandyTensor* positions, double theta, int32_t split_half,
                                const SandyTensor* q_out, char* err, size_t err_cap) {
    Err e{err, err_cap};
    int st = set_device(d, e);
    if (st) return st;
    std::lock_guard<std::mutex> lock(d->impl.mu);
    if (count > kQkvMaxRows) return fail(e, SANDY_ERR_UNSUPPORTED, "qkv matmul takes at most %d sequences", kQkvMaxRows);
    if (!valid_rank(lhs) || lhs->rank != 2 || lhs->dims[0] != count)
        return fail(e, SANDY_ERR_INVALID, "qkv matmul lhs must be [count, k]");
    // the kernel appends 2-byte elements at 16-bit page offsets; the page size
    // is a power of two (checked when the pool was made)
    uint32_t* errw = device_error_word(e, &st);
    if (st) return st;
    // checks that do not move bookkeeping first: the weight shape is checked
    // again by the GEMM, but a failure there must not leave lengths advanced
    auto kit = d->impl.pools.find(k_pool);
    if (kit != d->impl.pools.end()) {
        if (q_heads <= 0 || q_heads % kit->second->prefix != 0)
            return fail(e, SANDY_ERR_INVALID, "attention heads must be divisible by kv_heads");
        const int64_t n = (q_heads + 2 * kit->second->prefix) * kit->second->inner;
        if (!valid_rank(rhs) || rhs->rank != 2 || rhs->dims[0] != n || rhs->dims[1] != lhs->dims[1])
            return fail(e, SANDY_ERR_INVALID, "qkv matmul weight must be [(q_heads + 2 kv_heads) head_dim, k]");
        if (lhs->dtype != SANDY_BF16 || rhs->dtype != SANDY_BF16 || lhs->dims[1] % 32 != 0 || !contiguous(*lhs) ||
            !contiguous(*rhs) || ((reinterpret_cast<uintptr_t>(base_ptr(*lhs)) | reinterpret_cast<uintptr_t>(base_ptr(*rhs))) & 15u))
            return fail(e, SANDY_ERR_UNSUPPORTED, "qkv matmul needs contiguous 16-byte aligned bf16 operands, k a multiple of 32");
        // the GEMM's own checks (norm weight, row statistics, plan, workspace)
        // run dry before qkv_step moves any length
        QkvRope probe{};
        probe.hq = q_heads;
        probe.hkv = static_cast<int32_t>(kit->second->prefix);
        probe.d = static_cast<int32_t>(kit->second->inner);
        st = matmul_qkv(lhs, lhs_stats, norm_weight, eps, rhs, probe, d->impl.stream, e, true);
        if (st) return st;
    }
    for (uint32_t id : {k_pool, v_pool}) {
        auto it = d->impl.pools.find(id);
        if (it != d->impl.pools.end() &&
            static_cast<int64_t>(it->second->desc.max_tensors) * it->second->desc.max_blocks > 0x7fffffff)
            return fail(e, SANDY_ERR_UNSUPPORTED, "qkv matmul block tables exceed 32-bit indexing");
    }
    QkvStep q;
    st = qkv_step(d, k_pool, k_tensors, v_pool, v_tensors, count, q_heads, positions, theta, q_out, q, e);
    if (st) return st;
    QkvRope r{};
    PagedPool& kp = *q.kp;
    PagedPool& vp = *q.vp;
    r.q_out = static_cast<uint16_t*>(base_ptr(*q_out));
    r.k_pages = kp.pages;
    r.v_pages = vp.pages;
    r.k_table = kp.table;
    r.v_table = vp.table;
    r.k_len = kp.lengths;
    r.v_len = vp.lengths;
    r.k_max_blocks = static_cast<int32_t>(kp.desc.max_blocks);
    r.v_max_blocks = static_cast<int32_t>(vp.desc.max_blocks);
    r.page_bytes = static_cast<int64_t>(kp.page_elems * kp.elem);
    r.page_shift = 0;
    while ((int64_t{1} << r.page_shift) < kp.desc.page_size) r.page_shift++;
    r.hq = q_heads;
    r.hkv = static_cast<int32_t>(q.hkv);
    r.d = static_cast<int32_t>(q.D);
    r.split_half = split_half ? 1 : 0;
    r.pos = base_ptr(*positions);
    r.pos_dt = positions->dtype;
    r.errw = errw;
    const float th = static_cast<float>(theta);
    for (int i = 0; i < q.D / 2; i++) r.denom[i] = std::pow(th, static_cast<float>(2 * i) / static_cast<float>(q.D));
    std::copy(q.k_slots, q.k_slots + count, r.k_slots);
    std::copy(q.v_slots, q.v_slots + count, r.v_slots);
    return matmul_qkv(lhs, lhs_stats, norm_weight, eps, rhs, r, d->impl.stream, e);
}

namespace {
// out[i] = device length of tensors[i] + delta
int paged_lengths_plus(SandyHipDevice* d, uint32_t pool, const uint32_t* tensors, int32_t count,
                       const SandyTensor* positions, int32_t delta, Err e) {
    int st = set_device(d, e);
    if (st) return st;
    std::lock_guard<std::mutex> lock(d->impl.mu);
    auto pit = d->impl.pools.find(pool);
    if (pit == d->impl.pools.end()) return fail(e, SANDY_ERR_INVALID, "hip device paged pool not found");
    if (count <= 0 || count > kMaxStepTensors) return fail(e, SANDY_ERR_INVALID, "paged positions count out of range");
    if (!positions || !is_index(positions->dtype) || numel(*positions) != count || !contiguous(*positions))
        return fail(e, SANDY_ERR_INVALID, "paged positions output must be [count] i32 or i64");
    StepArgs args{};
    for (int i = 0; i < count; i++) {
        auto it = d->impl.tensors.find(tensors[i]);
        if (it == d->impl.tensors.end() || it->second.pool != pool)
            return fail(e, SANDY_ERR_INVALID, "hip device paged tensor not found");
        args.slots[i] = it->second.slot;
    }
    hipLaunchKernelGGL(paged_positions_kernel, dim3(static_cast<unsigned>((count + 255) / 256)), dim3(256), 0,
                       d->impl.stream, pit->second->lengths, base_ptr(*positions), positions->dtype, count, delta, args);
    SANDY_HIP_TRY(hipGetLastError(), e, "paged positions launch");
    return ok(e);
}
} // namespace

int sandy_hip_device_paged_positions(SandyHipDevice* d, uint32_t pool, const uint32_t* tensors, int32_t count,
                                     const SandyTensor* positions, char* err, size_t err_cap) {
    return paged_lengths_plus(d, pool, tensors, count, positions, -1, Err{err, err_cap});
}

int sandy_hip_device_paged_lengths(SandyHipDevice* d, uint32_t pool, const uint32_t* tensors, int32_t count,
                                   const SandyTensor* lengths, char* err, size_t err_cap) {
    return paged_lengths_plus(d, pool, tensors, count, lengths, 0, Err{err, err_cap});
}

int sandy_hip_device_paged_meta(SandyHipDevice* d, uint32_t tensor, SandyPagedMeta* meta, char* err, size_t err_cap) {
    Err e{err, err_cap};
    if (!d || !meta) return fail(e, SANDY_ERR_INVALID, "paged meta arguments are null");
    std::lock_guard<std::mutex> lock(d->impl.mu);
    auto it = d->impl.tensors.find(tensor);
    if (it == d->impl.tensors.end()) return fail(e, SANDY_ERR_INVALID, "hip device paged tensor not found");
    const PagedTensor& t = it->second;
    const PagedPool& p = *d->impl.pools.at(t.pool);
    *meta = SandyPagedMeta{};
    meta->pool = t.pool;
    meta->dtype = p.desc.dtype;
    meta->rank = p.desc.rank;
    meta->slot = t.slot;
    for (int i = 0; i < p.desc.rank; i++) meta->dims[i] = i == p.desc.grow_dim ? t.grow_length : p.desc.dims[i];
    meta->grow_dim = p.desc.grow_dim;
    meta->page_size = p.desc.page_size;
    meta->grow_length = t.grow_length;
    meta->page_count = static_cast<int64_t>(t.pages.size());
    meta->page_element_count = p.page_elems;
    return ok(e);
}

int sandy_hip_device_paged_read(SandyHipDevice* d, uint32_t tensor, void* host, uint64_t bytes, char* err,
                                size_t err_cap) {
    Err e{err, err_cap};
    int st = set_device(d, e);
    if (st) return st;
    std::lock_guard<std::mutex> lock(d->impl.mu);
    auto it = d->impl.tensors.find(tensor);
    if (it == d->impl.tensors.end()) return fail(e, SANDY_ERR_INVALID, "hip device paged tensor not found");
    const PagedTensor& t = it->second;
    const PagedPool& p = *d->impl.pools.at(t.pool);
    const size_t row = static_cast<size_t>(p.inner) * p.elem;
    const size_t need = static_cast<size_t>(p.prefix * t.grow_length) * row;
    if (bytes < need) return fail(e, SANDY_ERR_INVALID, "hip device paged read buffer too small");
    // CpuDevice.cpp:611-676: dense[prefix, grow, :] = page[prefix, grow % page_size, :]
    char* out = static_cast<char*>(host);
    SANDY_HIP_TRY(hipStreamSynchronize(d->impl.stream), e, "hipStreamSynchronize");
    for (int64_t pr = 0; pr < p.prefix; pr++) {
        for (int64_t g0 = 0; g0 < t.grow_length; g0 += p.desc.page_size) {
            const int64_t n = std::min<int64_t>(p.desc.page_size, t.grow_length - g0);
            const int32_t page = t.pages[static_cast<size_t>(g0 / p.desc.page_size)];
            const char* src = p.pages + (static_cast<int64_t>(page) * p.page_elems + pr * p.desc.page_size * p.inner) * p.elem;
            SANDY_HIP_TRY(hipMemcpy(out + (pr * t.grow_length + g0) * row, src, n * row, hipMemcpyDeviceToHost), e,
                          "paged read");
        }
    }
    return ok(e);
}

int sandy_hip_device_paged_views(SandyHipDevice* d, uint32_t pool, SandyPagedCache* cache, SandyTensor* block_table,
                                 SandyTensor* lengths, char* err, size_t err_cap) {
    Err e{err, err_cap};
    if (!d) return fail(e, SANDY_ERR_INVALID, "hip device is null");
    std::lock_guard<std::mutex> lock(d->impl.mu);
    auto pit = d->impl.pools.find(pool);
    if (pit == d->impl.pools.end()) return fail(e, SANDY_ERR_INVALID, "hip device paged pool not found");
    const PagedPool& p = *pit->second;
    if (cache) {
        *cache = SandyPagedCache{};
        cache->pool = p.pages;
        cache->dtype = p.desc.dtype;
        cache->page_size = p.desc.page_size;
        cache->prefix = p.prefix;
        cache->inner = p.inner;
        cache->num_pages = p.capacity;
    }
    if (block_table) {
        *block_table = SandyTensor{};
        block_table->data = p.table;
        block_table->dtype = SANDY_I32;
        block_table->rank = 2;
        block_table->dims[0] = p.desc.max_tensors;
        block_table->dims[1] = p.desc.max_blocks;
        block_table->strides[0] = p.desc.max_blocks;
        block_table->strides[1] = 1;
    }
    if (lengths) {
        *lengths = SandyTensor{};
        lengths->data = p.lengths;
        lengths->dtype = SANDY_I32;
        lengths->rank = 1;
        lengths->dims[0] = p.desc.max_tensors;
        lengths->strides[0] = 1;
    }
    return ok(e);
}

int sandy_hip_device_paged_sync(SandyHipDevice* d, uint32_t pool, char* err, size_t err_cap) {
    Err e{err, err_cap};
    int st = set_device(d, e);
    if (st) return st;
    std::lock_guard<std::mutex> lock(d->impl.mu);
    auto pit = d->impl.pools.find(pool);
    if (pit == d->impl.pools.end()) return fail(e, SANDY_ERR_INVALID, "hip device paged pool not found");
    PagedPool& p = *pit->second;
    std::vector<int32_t> lens(static_cast<size_t>(p.desc.max_tensors));
    SANDY_HIP_TRY(hipStreamSynchronize(d->impl.stream), e, "hipStreamSynchronize");
    SANDY_HIP_TRY(hipMemcpy(lens.data(), p.lengths, lens.size() * 4, hipMemcpyDeviceToHost), e, "length read");
    for (auto& t : d->impl.tensors)
        if (t.second.pool == pool) t.second.grow_length = lens[static_cast<size_t>(t.second.slot)];
    return ok(e);
}

int sandy_hip_device_graph_begin(SandyHipDevice* d, char* err, size_t err_cap) {
    Err e{err, err_cap};
    int st = set_device(d, e);
    if (st) return st;
    if (d->impl.capturing) return fail(e, SANDY_ERR_INVALID, "hip device is already capturing");
    SANDY_HIP_TRY(hipStreamBeginCapture(d->impl.stream, hipStreamCaptureModeThreadLocal), e, "hipStreamBeginCapture");
    d->impl.capturing = reinterpret_cast<hipGraph_t>(1);
    return ok(e);
}

int sandy_hip_device_graph_end(SandyHipDevice* d, uint32_t* graph, char* err, size_t err_cap) {
    Err e{err, err_cap};
    int st = set_device(d, e);
    if (st) return st;
    if (!d->impl.capturing) return fail(e, SANDY_ERR_INVALID, "hip device is not capturing");
    hipGraph_t g = nullptr;
    d->impl.capturing = nullptr;
    SANDY_HIP_TRY(hipStreamEndCapture(d->impl.stream, &g), e, "hipStreamEndCapture");
    hipGraphExec_t exec = nullptr;
    hipError_t rc = hipGraphInstantiate(&exec, g, nullptr, nullptr, 0);
    hipGraphDestroy(g);
    if (rc != hipSuccess) return fail(e, SANDY_ERR_HIP, "hipGraphInstantiate: %s", hipGetErrorString(rc));
    std::lock_guard<std::mutex> lock(d->impl.mu);
    const uint32_t id = d->impl.next_id++;
    d->impl.graphs[id] = exec;
    *graph = id;
    return ok(e);
}

int sandy_hip_device_graph_launch(SandyHipDevice* d, uint32_t graph, char* err, size_t err_cap) {
    Err e{err, err_cap};
    int st = set_device(d, e);
    if (st) return st;
    auto it = d->impl.graphs.find(graph);
    if (it == d->impl.graphs.end()) return fail(e, SANDY_ERR_INVALID, "hip device graph not found");
    SANDY_HIP_TRY(hipGraphLaunch(it->second, d->impl.stream), e, "hipGraphLaunch");
    return ok(e);
}

int sandy_hip_device_graph_destroy(SandyHipDevice* d, uint32_t graph, char* err, size_t err_cap) {
    Err e{err, err_cap};
    int st = set_device(d, e);
    if (st) return st;
    auto it = d->impl.graphs.find(graph);
    if (it == d->impl.graphs.end()) return fail(e, SANDY_ERR_INVALID, "hip device graph not found");
    SANDY_HIP_TRY(hipStreamSynchronize(d->impl.stream), e, "hipStreamSynchronize");
    hipGraphExecDestroy(it->second);
    d->impl.graphs.erase(it);
    return ok(e);
}

} // extern "C"
