// paged_operand.hip -- the reference's paged tensor as an operand of the
// non-attention kernel families.
//
// The reference hands a kernel a paged input as a page table plus the
// logical shape (CudaDeviceBufferView with paged = true, built in
// CudaDevice::run, src/device/cuda/CudaDevice.cpp:468-493) and every
// load_float / load_int of that operand resolves its page on each element
// (paged_storage_index, src/device/cuda/CudaKernelUtils.cuh:82-108).  Only
// inputs can be paged there (outputs must be dense tensor views,
// CudaDevice.cpp:497-503).
//
// Here a paged input of element-wise, norm, RoPE, softmax, reduction,
// embedding gather or attention (q, positions) is first gathered into a dense
// row-major copy by one kernel, and the family's dense kernel reads that copy.
// A page holds page_size rows of the grow dimension for every leading
// element, [prefix, page_size, inner], so one logical row of `inner` elements
// is contiguous in its page: the gather walks (prefix, grow row) rows with
// 16-byte pieces where row bytes and page addresses allow, elements
// otherwise.  Elements on pages the table does not have (ordinal >= page
// count, or a null page) read as zero, as load_float_at_storage returns 0 for
// them.  The copy is exact, so results equal the reference's in-place reads.
#include "common.h"

#include <bit>
#include <limits>

namespace sandy_hip {
namespace {

struct GatherArgs {
    const uint64_t* pages;
    char* out;
    int64_t rows;          // prefix * grow length
    int64_t grow;          // logical grow length
    int64_t row_bytes;     // inner * element size
    int64_t page_prefix_bytes;  // page_size * row_bytes: one leading element's slice of a page
    int64_t page_count;
    int32_t shift;         // log2 page_size
    int32_t pieces;        // 16-byte pieces per row (0: element copy)
    int32_t esize;
};

// One thread per 16-byte piece of a row (rows whose bytes are a multiple of
// 16 and whose pages are 16-byte aligned), consecutive threads on
// consecutive pieces of a row.
__global__ void __launch_bounds__(256) paged_gather16_kernel(GatherArgs a, int64_t total) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= total) return;
    const int64_t row = i / a.pieces;
    const int64_t piece = i - row * a.pieces;
    const int64_t prefix = row / a.grow;
    const int64_t g = row - prefix * a.grow;
    const int64_t ord = g >> a.shift;
    uint4 v = {0u, 0u, 0u, 0u};
    if (ord < a.page_count) {
        const uint64_t page = a.pages[ord];
        if (page != 0) {
            const int64_t at = prefix * a.page_prefix_bytes + (g & ((int64_t{1} << a.shift) - 1)) * a.row_bytes +
                               piece * 16;
            const char* p = reinterpret_cast<const char*>(page) + at;
            if ((page & 15u) == 0) {
                v = *reinterpret_cast<const uint4*>(p);
            } else {
                // a page address the reference's allocator would not give, still read exactly
                unsigned w[4] = {0u, 0u, 0u, 0u};
                for (int j = 0; j < 16; j++)
                    w[j >> 2] |= static_cast<unsigned>(static_cast<unsigned char>(p[j])) << (8 * (j & 3));
                v = uint4{w[0], w[1], w[2], w[3]};
            }
        }
    }
    *reinterpret_cast<uint4*>(a.out + row * a.row_bytes + piece * 16) = v;
}

// One thread per element (any row width or page alignment).
template <typename W>
__global__ void __launch_bounds__(256) paged_gather_elems_kernel(GatherArgs a, int64_t total) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= total) return;
    const int64_t per_row = a.row_bytes / static_cast<int64_t>(sizeof(W));
    const int64_t row = i / per_row;
    const int64_t inner = i - row * per_row;
    const int64_t prefix = row / a.grow;
    const int64_t g = row - prefix * a.grow;
    const int64_t ord = g >> a.shift;
    W v = W(0);
    if (ord < a.page_count) {
        const uint64_t page = a.pages[ord];
        if (page != 0) {
            const int64_t at = prefix * a.page_prefix_bytes + (g & ((int64_t{1} << a.shift) - 1)) * a.row_bytes +
                               inner * static_cast<int64_t>(sizeof(W));
            v = *reinterpret_cast<const W*>(reinterpret_cast<const char*>(page) + at);
        }
    }
    reinterpret_cast<W*>(a.out)[i] = v;
}

// The checks of pack_tensor_arg for a paged buffer (CudaKernelUtils.cuh:
// 290-374), worded for this backend.
int check_paged(const SandyPagedTensor* t, Err e, int64_t* numel_out, int64_t* inner_out) {
    if (!t) return fail(e, SANDY_ERR_INVALID, "hip paged tensor is null");
    if (t->rank < 1 || t->rank > SANDY_HIP_MAX_RANK) return fail(e, SANDY_ERR_INVALID, "hip tensor rank exceeds kernel max rank");
    if (dtype_size(t->dtype) == 0 || t->dtype == SANDY_F16 || t->dtype == SANDY_U8)
        return fail(e, SANDY_ERR_INVALID, "hip paged tensor unsupported dtype");
    if (t->grow_dim < 0 || t->grow_dim >= t->rank) return fail(e, SANDY_ERR_INVALID, "hip paged tensor grow_dim out of range");
    if (t->page_size <= 0) return fail(e, SANDY_ERR_INVALID, "hip paged tensor page_size must be > 0");
    if (!std::has_single_bit(static_cast<uint64_t>(t->page_size)))
        return fail(e, SANDY_ERR_INVALID, "hip paged tensor page_size must be a power of two");
    if (t->page_count < 0) return fail(e, SANDY_ERR_INVALID, "hip paged tensor page_count must be >= 0");
    int64_t n = 1;
    for (int i = 0; i < t->rank; i++) {
        if (t->dims[i] < 0) return fail(e, SANDY_ERR_INVALID, "hip tensor dim must be static");
        if (t->dims[i] > 0 && n > std::numeric_limits<int64_t>::max() / t->dims[i])
            return fail(e, SANDY_ERR_INVALID, "hip paged tensor element count overflow");
        n *= t->dims[i];
    }
    int64_t inner = 1;
    for (int i = static_cast<int>(t->grow_dim) + 1; i < t->rank; i++) {
        if (t->dims[i] <= 0) return fail(e, SANDY_ERR_INVALID, "hip paged tensor inner dimensions must be positive");
        if (inner > std::numeric_limits<int64_t>::max() / t->dims[i])
            return fail(e, SANDY_ERR_INVALID, "hip paged tensor inner element count overflow");
        inner *= t->dims[i];
    }
    if (inner > std::numeric_limits<int64_t>::max() / t->page_size / 8)
        return fail(e, SANDY_ERR_INVALID, "hip paged tensor physical prefix size overflow");
    if (n != 0 && !t->pages) return fail(e, SANDY_ERR_INVALID, "hip paged tensor page table is null");
    *numel_out = n;
    *inner_out = inner;
    return SANDY_OK;
}

int gather(const SandyPagedTensor* src, void* dst, hipStream_t stream, Err e) {
    int64_t n = 0, inner = 0;
    int st = check_paged(src, e, &n, &inner);
    if (st) return st;
    if (n == 0) return ok(e);
    const int64_t es = static_cast<int64_t>(dtype_size(src->dtype));
    GatherArgs a{};
    a.pages = static_cast<const uint64_t*>(src->pages);
    a.out = static_cast<char*>(dst);
    a.grow = src->dims[src->grow_dim];
    a.rows = n / inner;
    a.row_bytes = inner * es;
    a.page_prefix_bytes = src->page_size * a.row_bytes;
    a.page_count = src->page_count;
    a.shift = std::countr_zero(static_cast<uint64_t>(src->page_size));
    a.esize = static_cast<int32_t>(es);
    // 16-byte pieces where every row offset inside a page is a multiple of 16
    // (the page addresses are device data: an unaligned page is read bytewise)
    const bool vec = a.row_bytes % 16 == 0 && (reinterpret_cast<uintptr_t>(dst) & 15u) == 0 &&
                     a.row_bytes / 16 <= 0x7fffffff;
    const int64_t total = vec ? a.rows * (a.row_bytes / 16) : n;
    const int64_t blocks = (total + 255) / 256;
    if (blocks > 0x7fffffff) return fail(e, SANDY_ERR_UNSUPPORTED, "hip paged tensor exceeds the launch grid");
    if (vec) {
        a.pieces = static_cast<int32_t>(a.row_bytes / 16);
        hipLaunchKernelGGL(paged_gather16_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, a, total);
    } else if (es == 2) {
        hipLaunchKernelGGL(paged_gather_elems_kernel<uint16_t>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, a, total);
    } else if (es == 4) {
        hipLaunchKernelGGL(paged_gather_elems_kernel<uint32_t>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, a, total);
    } else {
        hipLaunchKernelGGL(paged_gather_elems_kernel<uint64_t>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, a, total);
    }
    SANDY_HIP_TRY(hipGetLastError(), e, "paged gather");
    return ok(e);
}

void dense_desc(const SandyPagedTensor* src, void* data, SandyTensor* out) {
    *out = SandyTensor{};
    out->data = data;
    out->dtype = src->dtype;
    out->rank = src->rank;
    int64_t s = 1;
    for (int i = src->rank - 1; i >= 0; i--) {
        out->dims[i] = src->dims[i];
        out->strides[i] = s;
        s *= src->dims[i];
    }
}

} // namespace
} // namespace sandy_hip

using namespace sandy_hip;

extern "C" int sandy_hip_paged_to_dense(const SandyPagedTensor* src, const SandyTensor* dst, void* stream, char* err,
                                        size_t err_cap) {
    Err e{err, err_cap};
    int64_t n = 0, inner = 0;
    int st = check_paged(src, e, &n, &inner);
    if (st) return st;
    if (!valid_rank(dst) || dst->dtype != src->dtype || dst->rank != src->rank || !contiguous(*dst))
        return fail(e, SANDY_ERR_INVALID, "hip paged tensor destination must be a contiguous tensor of its shape and dtype");
    for (int i = 0; i < src->rank; i++)
        if (dst->dims[i] != src->dims[i])
            return fail(e, SANDY_ERR_INVALID, "hip paged tensor destination must be a contiguous tensor of its shape and dtype");
    if (n != 0 && !dst->data) return fail(e, SANDY_ERR_INVALID, "hip paged tensor destination is null");
    return gather(src, base_ptr(*dst), static_cast<hipStream_t>(stream), e);
}

extern "C" int sandy_hip_paged_stage(const SandyPagedTensor* src, int32_t slot, SandyTensor* dense, void* stream,
                                     char* err, size_t err_cap) {
    Err e{err, err_cap};
    if (slot < 0 || slot >= SANDY_HIP_PAGED_STAGE_SLOTS)
        return fail(e, SANDY_ERR_INVALID, "hip paged stage slot out of range");
    if (!dense) return fail(e, SANDY_ERR_INVALID, "hip paged stage needs an output descriptor");
    int64_t n = 0, inner = 0;
    int st = check_paged(src, e, &n, &inner);
    if (st) return st;
    const size_t bytes = static_cast<size_t>(n) * dtype_size(src->dtype);
    void* ws = device_workspace(kPagedStageSlot0 + slot, bytes, static_cast<hipStream_t>(stream), e, &st);
    if (st) return st;
    dense_desc(src, ws, dense);
    return gather(src, ws, static_cast<hipStream_t>(stream), e);
}
