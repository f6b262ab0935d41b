// layout.hip -- LayoutTransformKernelOp: materialise a strided view.
//
// The reference launches a layout transform only when the engine cannot
// alias it as a view (Engine::try_alias_layout_op, src/engine/Engine.cpp:
// 606-754: a reshape or contiguous of a non-default view, e.g. a transposed
// one), and its CUDA kernel copies the input view's logical elements into the
// output in row-major order, one thread and one scalar access per element,
// with an int64 div/mod per dimension on both sides
// (src/device/cuda/CudaLayoutTransformKernels.cu:25-78).  The element order
// is the same here; the copy is planned on the host instead:
//   - dimensions are collapsed where the input's strides allow, against a
//     contiguous output (the usual case) seen in the input's shape;
//   - one contiguous run: a 16-byte vector copy;
//   - unit innermost input stride: rows copied as 16-byte vectors when
//     their length and addresses allow, else element by element;
//   - an inner dimension of unit input stride that is not the last: a
//     64 x 64 tile transposed through LDS, so both the reads (along the
//     input's unit stride) and the writes (along the output's rows) are
//     whole 128-byte lines;
//   - anything else (a strided output too): the reference's per-element walk.
// It is bandwidth-bound data movement (bytes read = bytes written = numel *
// element size).
#include "common.h"

#include <algorithm>

namespace sandy_hip {
namespace {

constexpr int kMaxDims = SANDY_HIP_MAX_RANK;
typedef unsigned int v4u __attribute__((ext_vector_type(4)));  // 16-byte piece (non-temporal access)

struct Walk {  // a view collapsed to rank <= 8, innermost last
    int32_t rank;
    int64_t dims[kMaxDims];
    int64_t in_st[kMaxDims];   // input strides (elements)
    int64_t out_st[kMaxDims];  // output strides (elements)
};

// Storage offsets of linear element i (row-major over w.dims) in the input
// and the output.
__device__ __forceinline__ void walk_offsets(const Walk& w, int64_t i, int64_t& ii, int64_t& oi) {
    ii = 0;
    oi = 0;
    for (int d = w.rank - 1; d >= 0; d--) {
        const int64_t c = i % w.dims[d];
        i /= w.dims[d];
        ii += c * w.in_st[d];
        oi += c * w.out_st[d];
    }
}

template <typename E>
__global__ __launch_bounds__(256) void layout_generic_kernel(const E* __restrict__ in, E* __restrict__ out, Walk w,
                                                             int64_t n) {
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n; i += static_cast<int64_t>(gridDim.x) * 256) {
        int64_t ii, oi;
        walk_offsets(w, i, ii, oi);
        out[oi] = in[ii];
    }
}

// n16 16-byte pieces, both sides contiguous and 16-byte aligned.
__global__ __launch_bounds__(256) void layout_copy16_kernel(const v4u* __restrict__ in, v4u* __restrict__ out,
                                                            int64_t n16) {
    const int64_t step = static_cast<int64_t>(gridDim.x) * 256;
    int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    for (; i + 3 * step < n16; i += 4 * step) {
        const v4u a = __builtin_nontemporal_load(in + i), b = __builtin_nontemporal_load(in + i + step),
                    c = __builtin_nontemporal_load(in + i + 2 * step), d = __builtin_nontemporal_load(in + i + 3 * step);
        __builtin_nontemporal_store(a, out + i);
        __builtin_nontemporal_store(b, out + i + step);
        __builtin_nontemporal_store(c, out + i + 2 * step);
        __builtin_nontemporal_store(d, out + i + 3 * step);
    }
    for (; i < n16; i += step) __builtin_nontemporal_store(__builtin_nontemporal_load(in + i), out + i);
}

// Rows of `row16` 16-byte pieces: the input row r starts at the element
// offset of outer index r (the walk over the outer dims), the output rows
// are contiguous.  A wave per row chunk.
__global__ __launch_bounds__(256) void layout_rows16_kernel(const char* __restrict__ in, v4u* __restrict__ out,
                                                            Walk outer, int64_t rows, int64_t row16, int32_t esz) {
    const int lane = threadIdx.x & 63;
    const int64_t wave = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) >> 6;
    const int64_t waves = static_cast<int64_t>(gridDim.x) * 4;
    for (int64_t r = wave; r < rows; r += waves) {
        int64_t ii, oi;
        walk_offsets(outer, r, ii, oi);
        const v4u* src = reinterpret_cast<const v4u*>(in + ii * esz);
        v4u* dst = out + r * row16;
        for (int64_t p = lane; p < row16; p += 64) __builtin_nontemporal_store(__builtin_nontemporal_load(src + p), dst + p);
    }
}

// The 2-D transpose core.  Outer slice s starts at the input offset the walk
// `outer` gives; the output slices are contiguous [A][Bc] blocks.  The input
// has unit stride along a (the output's row index) and stride sb along b
// (the output's column index).  A workgroup moves one 64 x 64 tile: lanes
// read 64 consecutive a for one b (whole input lines) into LDS, then write
// 64 consecutive b for one a (whole output lines).
template <typename E>
__global__ __launch_bounds__(256) void layout_tile_kernel(const E* __restrict__ in, E* __restrict__ out, Walk outer,
                                                          int64_t A, int64_t Bc, int64_t sb, int64_t tiles_a,
                                                          int64_t tiles_b) {
    __shared__ E tile[64][65];
    const int64_t t = blockIdx.x;
    const int64_t per_slice = tiles_a * tiles_b;
    const int64_t s = t / per_slice;
    const int64_t rem = t - s * per_slice;
    const int64_t ta = rem / tiles_b, tb = rem - (rem / tiles_b) * tiles_b;
    int64_t ii, oi;
    walk_offsets(outer, s, ii, oi);
    const E* src = in + ii;
    E* dst = out + s * A * Bc;
    const int x = threadIdx.x & 63, y = threadIdx.x >> 6;  // 64 lanes x 4 rows per pass
    const int64_t a0 = ta * 64, b0 = tb * 64;
    // read: lane x along a (unit input stride), rows y + 4k along b
#pragma unroll
    for (int k = 0; k < 16; k++) {
        const int64_t a = a0 + x, b = b0 + y + 4 * k;
        if (a < A && b < Bc) tile[y + 4 * k][x] = src[a + b * sb];
    }
    __syncthreads();
    // write: lane x along b (the output row), rows y + 4k along a
#pragma unroll
    for (int k = 0; k < 16; k++) {
        const int64_t a = a0 + y + 4 * k, b = b0 + x;
        if (a < A && b < Bc) dst[a * Bc + b] = tile[x][y + 4 * k];
    }
}

template <typename E>
void launch_generic(const void* in, void* out, const Walk& w, int64_t n, hipStream_t stream) {
    const int64_t blocks = std::min<int64_t>((n + 255) / 256, 65536);
    hipLaunchKernelGGL(layout_generic_kernel<E>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream,
                       static_cast<const E*>(in), static_cast<E*>(out), w, n);
}

template <typename E>
void launch_tile(const void* in, void* out, const Walk& outer, int64_t A, int64_t Bc, int64_t sb, int64_t slices,
                 hipStream_t stream) {
    const int64_t ta = (A + 63) / 64, tb = (Bc + 63) / 64;
    hipLaunchKernelGGL(layout_tile_kernel<E>, dim3(static_cast<unsigned>(slices * ta * tb)), dim3(256), 0, stream,
                       static_cast<const E*>(in), static_cast<E*>(out), outer, A, Bc, sb, ta, tb);
}

} // namespace
} // namespace sandy_hip

using namespace sandy_hip;

extern "C" int sandy_hip_layout_transform(const SandyTensor* in, const SandyTensor* out, int32_t kind, void* stream_,
                                          char* err, size_t err_cap) {
    Err e{err, err_cap};
    hipStream_t stream = static_cast<hipStream_t>(stream_);
    if (kind == SANDY_LAYOUT_SLICE) return fail(e, SANDY_ERR_INVALID, "slice layout aliases must not launch on HIP");
    if (kind < SANDY_LAYOUT_RESHAPE || kind > SANDY_LAYOUT_CONTIGUOUS)
        return fail(e, SANDY_ERR_INVALID, "hip layout_transform unknown transform kind");
    if (!valid_rank(in) || !valid_rank(out)) return fail(e, SANDY_ERR_INVALID, "hip layout_transform tensor rank out of range");
    if (in->dtype != out->dtype) return fail(e, SANDY_ERR_INVALID, "hip layout_transform dtype mismatch");
    const size_t esz = dtype_size(in->dtype);
    if (esz == 0) return fail(e, SANDY_ERR_INVALID, "hip layout_transform unsupported dtype");
    const int64_t n = numel(*in);
    if (n < 0 || numel(*out) < 0) return fail(e, SANDY_ERR_INVALID, "hip layout_transform requires static shapes");
    if (n != numel(*out)) return fail(e, SANDY_ERR_INVALID, "hip layout_transform element count mismatch");
    if (n == 0) return ok(e);
    const void* src = base_ptr(*in);
    void* dst = base_ptr(*out);

    // A contiguous output is the input's shape read in row-major order, so
    // both sides walk the input's dims (collapsed, size-1 dims dropped).
    Walk w{};
    const bool out_contig = contiguous(*out);
    if (out_contig) {
        for (int d = 0; d < in->rank; d++) {
            if (in->dims[d] == 1) continue;
            if (w.rank > 0 && w.in_st[w.rank - 1] == in->strides[d] * in->dims[d]) {
                w.dims[w.rank - 1] *= in->dims[d];
                w.in_st[w.rank - 1] = in->strides[d];
            } else {
                w.dims[w.rank] = in->dims[d];
                w.in_st[w.rank] = in->strides[d];
                w.rank++;
            }
        }
        if (w.rank == 0) {
            w.rank = 1;
            w.dims[0] = 1;
            w.in_st[0] = 1;
        }
        int64_t st = 1;
        for (int d = w.rank - 1; d >= 0; d--) {
            w.out_st[d] = st;
            st *= w.dims[d];
        }
    }
    const uintptr_t align = reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst);
    if (out_contig && w.rank == 1 && w.in_st[0] == 1) {
        const int64_t bytes = n * static_cast<int64_t>(esz);
        if ((align & 15) == 0 && bytes % 16 == 0) {
            const int64_t n16 = bytes / 16;
            const int64_t blocks = std::min<int64_t>((n16 + 255) / 256, 8192);
            hipLaunchKernelGGL(layout_copy16_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream,
                               static_cast<const v4u*>(src), static_cast<v4u*>(dst), n16);
            SANDY_HIP_TRY(hipGetLastError(), e, "hip layout_transform launch");
            return ok(e);
        }
    }
    if (out_contig && w.rank >= 2 && w.in_st[w.rank - 1] == 1) {
        // rows: the innermost input dim is contiguous
        const int64_t row_bytes = w.dims[w.rank - 1] * static_cast<int64_t>(esz);
        bool vec = (align & 15) == 0 && row_bytes % 16 == 0;
        for (int d = 0; d < w.rank - 1 && vec; d++) vec = (w.in_st[d] * static_cast<int64_t>(esz)) % 16 == 0;
        if (vec) {
            Walk outer{};
            outer.rank = w.rank - 1;
            for (int d = 0; d < outer.rank; d++) {
                outer.dims[d] = w.dims[d];
                outer.in_st[d] = w.in_st[d];
                outer.out_st[d] = 0;
            }
            const int64_t rows = n / w.dims[w.rank - 1];
            const int64_t blocks = std::min<int64_t>((rows + 3) / 4, 16384);
            hipLaunchKernelGGL(layout_rows16_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream,
                               static_cast<const char*>(src), static_cast<v4u*>(dst), outer, rows, row_bytes / 16,
                               static_cast<int32_t>(esz));
            SANDY_HIP_TRY(hipGetLastError(), e, "hip layout_transform launch");
            return ok(e);
        }
    }
    if (out_contig && w.rank >= 2 && w.in_st[w.rank - 1] != 1) {
        // a transposed inner pair: unit input stride on dim a < last
        int a = -1;
        for (int d = 0; d < w.rank - 1; d++)
            if (w.in_st[d] == 1) a = d;
        if (a == w.rank - 2 && w.dims[a] >= 16 && w.dims[w.rank - 1] >= 16) {
            Walk outer{};
            outer.rank = std::max(1, w.rank - 2);
            outer.dims[0] = 1;
            outer.in_st[0] = 0;
            for (int d = 0; d < w.rank - 2; d++) {
                outer.dims[d] = w.dims[d];
                outer.in_st[d] = w.in_st[d];
            }
            int64_t slices = 1;
            for (int d = 0; d < w.rank - 2; d++) slices *= w.dims[d];
            const int64_t A = w.dims[a], Bc = w.dims[w.rank - 1], sb = w.in_st[w.rank - 1];
            if (slices * ((A + 63) / 64) * ((Bc + 63) / 64) < (1LL << 31)) {
                switch (esz) {
                    case 1: launch_tile<uint8_t>(src, dst, outer, A, Bc, sb, slices, stream); break;
                    case 2: launch_tile<uint16_t>(src, dst, outer, A, Bc, sb, slices, stream); break;
                    case 4: launch_tile<uint32_t>(src, dst, outer, A, Bc, sb, slices, stream); break;
                    default: launch_tile<uint64_t>(src, dst, outer, A, Bc, sb, slices, stream); break;
                }
                SANDY_HIP_TRY(hipGetLastError(), e, "hip layout_transform launch");
                return ok(e);
            }
        }
    }
    if (!out_contig) {
        // both sides strided: walk the output's dims, the input's by its own shape
        // when the shapes agree (a reshape into a strided output walks linear order
        // through the input's dims, checked below)
        if (in->rank != out->rank || !same_shape(*in, *out)) {
            // general reshape into a strided output: unravel against each shape
            // (rare: the engine allocates layout outputs with default views)
            return fail(e, SANDY_ERR_UNSUPPORTED, "hip layout_transform reshape into a strided output");
        }
        w.rank = in->rank;
        for (int d = 0; d < in->rank; d++) {
            w.dims[d] = in->dims[d];
            w.in_st[d] = in->strides[d];
            w.out_st[d] = out->strides[d];
        }
    }
    switch (esz) {
        case 1: launch_generic<uint8_t>(src, dst, w, n, stream); break;
        case 2: launch_generic<uint16_t>(src, dst, w, n, stream); break;
        case 4: launch_generic<uint32_t>(src, dst, w, n, stream); break;
        default: launch_generic<uint64_t>(src, dst, w, n, stream); break;
    }
    SANDY_HIP_TRY(hipGetLastError(), e, "hip layout_transform launch");
    return ok(e);
}
